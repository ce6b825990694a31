"""The C++ host API (tropical-gemm_amd/cpp/tropical_gemm_hip.hpp), the C++
counterpart of the reference's Rust GPU crate, exercised by the compiled test
program tests/cpp/test_hip_api (built by __graft_entry__.build())."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_hip_api")


def _run(mode: str) -> str:
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built; run __graft_entry__.build()")
    r = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout
    return r.stdout


def test_cpp_api_host_checks():
    out = _run("cpu")
    assert "cpu checks" in out


@pytest.mark.gpu
def test_cpp_api_on_gpu():
    out = _run("gpu")
    print(out)
    assert "gpu checks" in out
