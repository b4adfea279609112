"""CPU model of the decode kernels' grid barrier (tests/barrier_model.cpp).

The model compiles the protocol the device code uses (homelab_amd/csrc/grid_barrier.hpp:
monotonic arrival and exit counters per group, bases read from the exit counters at
kernel start, one add to arrive and one to exit) with one std::thread per block, started
in whatever order the OS runs them. It checks, on one shared barrier header: calls of 1 to
512 blocks in any order (every meeting releases, none early, no wait gives up); meetings
back to back on one area, with and without work between; that after a call whose waits
gave up (a late block, a tiny spin limit) the header serves the next call normally; and
that a block that starts only after every other block has arrived still reads the call's
bases (nobody gives up or passes early). It also runs the round-one protocol, which published the
generation to the first min(blocks, 8) words only, to show the model finds the fault that
form had after a call of fewer than 8 blocks.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "barrier_model.cpp")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = str(tmp_path_factory.mktemp("barrier") / "barrier_model")
    subprocess.run([gxx, "-O2", "-std=c++17", "-pthread", "-o", exe, SRC], check=True)
    return exe


@pytest.mark.parametrize("scenario", ["sizes", "twice", "b2b", "giveup", "giveup2", "late"])
def test_barrier_protocol(model, scenario):
    r = subprocess.run([model, scenario], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, f"{scenario}: rc {r.returncode}\n{r.stdout}"


def test_model_finds_the_partial_publication_fault(model):
    # the previous protocol: a call after one of fewer than 8 blocks gives up its waits
    r = subprocess.run([model, "old_sizes"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 1, f"the model did not find the fault:\n{r.stdout}"
    assert "gave up" in r.stdout
