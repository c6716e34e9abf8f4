"""The C++ host mirror (ssd-llm_amd/host/ssdq_compute.hpp: GpuCompute with the
MetalCompute surface, compute.rs:47-264, and the streamer.rs / block_swap.rs
helpers) driven from C++ on the GPU and checked against the oracle."""
import os
import subprocess

import pytest

from helpers import announce

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(__file__), "cpp", "test_host_mirror")


def test_host_mirror_binary():
    assert os.path.exists(BIN), "tests/cpp/test_host_mirror is not built (run __graft_entry__.build())"
    announce("C++ host mirror")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout
