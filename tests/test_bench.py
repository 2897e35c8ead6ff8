"""bench.py's host logic, no GPU: the rocprofv3 counter passes stay within
what one pass can collect on gfx950 (more in any block hangs the
profiler), the plan's byte fields parse, and a run on more than one GPU is
refused with a message."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

# counters one pass may hold, per block (FETCH_SIZE takes 3 TCC
# counters, WRITE_SIZE 2)
LIMITS = {"SQ": 8, "TCC": 4, "TCP": 4, "TA": 2, "TD": 2, "GRBM": 2}
COST = {"FETCH_SIZE": ("TCC", 3), "WRITE_SIZE": ("TCC", 2)}


def block_of(counter):
    if counter in COST:
        return COST[counter]
    return counter.split("_")[0], 1


@pytest.mark.parametrize("config", ["rows", "saxpy", "scatter", "poly", "mc", "mc64", "mc_greeks", "matmul",
                                    "matmul64", "bs_greeks"])
def test_counter_passes_fit_one_pass_each(config):
    for group in bench.counter_passes(config):
        used = {}
        for c in group:
            b, n = block_of(c)
            used[b] = used.get(b, 0) + n
        for b, n in used.items():
            assert b in LIMITS, (config, c)
            assert n <= LIMITS[b], (config, group)
        if any(c.startswith("SQ_") for c in group):
            assert "GRBM_GUI_ACTIVE" in group, group


def test_plan_bytes_carry_root_and_moved_bytes():
    from cudacaml_amd import backend_hip as H
    from cudacaml_amd.examples import configs as C

    pb = bench.plan_bytes(H, C.saxpy(1 << 20))
    assert {r for r, _, _ in pb.values()} == {"map", "reduce_split_fold"}
    # the sum folded in the map: its last fold keeps the root's bytes and
    # moves only its output
    folds = [(b, m) for r, b, m in pb.values() if r == "reduce_split_fold" and b > 0]
    assert folds == [(4 * (1 << 20) + 4, 4)]
    assert all(m <= b for _, b, m in pb.values())


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
