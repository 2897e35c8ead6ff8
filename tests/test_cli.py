"""The command line (bin/main.ml:1-61): list, emit, plan, dot without a
device; run and info on the device; check (tests/check.py, since it needs
the interpreter) with the reference's output and exit codes."""

import subprocess
import sys

import pytest

from cudacaml_amd.examples import programs


def cli(*args):
    return subprocess.run([sys.executable, "-m", "cudacaml_amd", *args], capture_output=True, text=True, timeout=120)


def test_list_names_every_example():
    r = cli("list")
    assert r.returncode == 0
    assert r.stdout.split() == [e.name for e in programs.all_examples()]


def test_emit_plan_dot():
    r = cli("emit", "chain")
    assert r.returncode == 0 and 'extern "C" __global__' in r.stdout
    r = cli("plan", "saxpy")
    assert r.returncode == 0 and r.stdout.startswith("program saxpy")
    r = cli("dot", "saxpy")
    assert r.returncode == 0 and r.stdout.startswith('digraph "saxpy"')


def test_unknown_example_and_usage():
    assert cli("emit", "nope").returncode == 2
    assert cli("bogus").returncode == 2
    r = cli("check", "saxpy")
    assert r.returncode == 2 and "tests/check.py saxpy" in r.stderr


def check_tool(*args):
    import os

    tool = os.path.join(os.path.dirname(os.path.abspath(__file__)), "check.py")
    return subprocess.run([sys.executable, tool, *args], capture_output=True, text=True, timeout=300)


def test_check_tool_usage_and_unknown_example():
    assert check_tool().returncode == 2
    r = check_tool("nope")
    assert r.returncode == 2 and "unknown example: nope" in r.stderr


def test_check_tool_verdicts_with_fake_candidates():
    """bin/main.ml:52-60 on the CPU: a candidate that agrees prints
    "<name>: ok" (exit 0); one that is 0.1% off prints "<name>: MISMATCH"
    with the output named (exit 1). The candidates wrap the oracle."""
    import io

    import check
    import oracle
    from test_differential import Slight

    e = programs.find("saxpy")
    out, err = io.StringIO(), io.StringIO()
    assert check.check_one(e, oracle.Interp, oracle.Interp, out, err) == 0
    assert out.getvalue() == "saxpy: ok\n"
    out, err = io.StringIO(), io.StringIO()
    assert check.check_one(e, oracle.Interp, Slight, out, err) == 1
    assert err.getvalue().startswith("saxpy: MISMATCH output r[1]")
    assert check.main(["saxpy"], candidate=Slight) == 1


@pytest.mark.gpu
def test_run_and_info(device):
    r = cli("run", "saxpy")
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith("r [1024] = [") and "\ns [] = [" in r.stdout
    r = cli("info")
    assert r.returncode == 0 and "compute: gfx950" in r.stdout


@pytest.mark.gpu
def test_check_tool_on_the_device(device):
    """check <example> against Backend_hip, and check all."""
    r = check_tool("saxpy")
    assert r.returncode == 0 and r.stdout == "saxpy: ok\n", r.stderr
    r = check_tool("all")
    assert r.returncode == 0, r.stderr
    assert r.stdout.splitlines() == ["%s: ok" % e.name for e in programs.all_examples()]
