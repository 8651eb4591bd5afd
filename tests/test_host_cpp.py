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


def _write_synth_gguf(path, seed):
    """A GGUF holding every tensor of a model synthesized on the device."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import gguf_writer as gw
    import make_golden
    from hearth_amd import Ctx, Model
    ctx = Ctx(0)
    m = Model(ctx, make_golden.DENSE)
    m.synthesize(seed)
    tensors = []
    for name, t, ne0, ne1, nb in m.tensors():
        shape = (ne0,) if ne1 == 1 and t == 0 else (ne0, ne1)
        tensors.append((name, t, shape, m.download(name, nb).tobytes()))
    gw.write_gguf(path, gw.model_meta(m.cfg), tensors)
    m.close()
    ctx.close()


@pytest.mark.gpu
def test_host_gpu_tests(tmp_path):
    path = str(tmp_path / "dense.gguf")
    _write_synth_gguf(path, 7)
    p = _run(["--gguf", path, "--seed", "7"], 600)
    print(p.stdout)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "FAIL" not in p.stdout and " 0 failed" in p.stdout, p.stdout
