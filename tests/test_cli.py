"""The command line (bin/main.ml:1-61): list, emit, plan, dot without a
device; check points at the parity suite; run and info on the device."""

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
    assert r.returncode == 2 and "tests/test_gpu_parity.py -k saxpy" in r.stderr


@pytest.mark.gpu
def test_run_and_info(device):
    r = cli("run", "saxpy")
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith("r [1024] = [") and "\ns [] = [" in r.stdout
    r = cli("info")
    assert r.returncode == 0 and "compute: gfx950" in r.stdout
