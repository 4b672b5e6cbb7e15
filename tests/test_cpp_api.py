"""The C++ operator API (include/atlas_neural_ops.hpp) through its test
program tests/cpp/neural_ops_test (built by __graft_entry__.build()):
the reference's NeuralOps known answers and tolerances
(crates/atlas-ops/tests/phase_02_operators.rs), bit-exact checks against the
oracle, the InvalidInput predicates, one resident call, the argmax tie KAT
(crates/atlas-metal/src/lib.rs:2217-2230), and the C++ GgufModel
(include/atlas_gguf.hpp) on the reference's GGUF reader tests
(crates/atlas-core/tests/phase_11a_gguf.rs:99-120), which need no device."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "neural_ops_test")


def run(*args, timeout=120):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built: run __graft_entry__.build()")
    return subprocess.run([BIN, *args], capture_output=True, text=True, timeout=timeout)


def test_cpp_api_reports_no_device_like_the_reference():
    """Without a GPU, NeuralOps construction raises NoDevice and the program
    skips its device assertions (require_ops, phase_02_operators.rs:8-19);
    with one, every check must pass."""
    import atlas_amd
    from ctypes import byref, c_int
    n = c_int()
    atlas_amd.load().atlas_hip_device_count(byref(n))
    p = run()
    assert p.returncode == 0, p.stderr
    if n.value == 0:
        assert "no HIP device" in p.stderr


@pytest.mark.gpu
def test_cpp_api_on_device():
    p = run("--require-device")
    print(p.stderr)
    assert p.returncode == 0, p.stderr
    assert "all operator checks passed" in p.stderr
