"""The C++ host side (hearth_amd/host/hearth_host.hpp: GpuCompute, Model,
Result) through its own test program, tests/cpp/test_host.cpp, which
__graft_entry__.build() compiles.  The program restates the reference's inline
tests for this path (q8_0.rs round trip, q2_0.rs / q1_0g128.rs known answers and
paired-vs-single fixtures, hearth-sampler greedy tests) and checks the model
calls against the CPU oracle.  --cpu runs the tests that need no device."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_host")


def _run(args, timeout):
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/test_host is not built: run __graft_entry__.build()")
    return subprocess.run([BIN] + args, capture_output=True, text=True, timeout=timeout)


def test_host_cpu_tests():
    p = _run(["--cpu"], 120)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "FAIL" not in p.stdout and " 0 failed" in p.stdout, p.stdout


@pytest.mark.gpu
def test_host_gpu_tests():
    p = _run([], 600)
    print(p.stdout)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "FAIL" not in p.stdout and " 0 failed" in p.stdout, p.stdout
