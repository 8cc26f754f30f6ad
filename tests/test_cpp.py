"""The C++ host mirror (staleynet_amd/host/staleynet_cuda.hpp) and the
reference's GPU parity test restated with it (tests/cpp)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCE = os.path.join(ROOT, "tests", "cpp", "kernels_match_reference.cpp")
BINARY = os.path.join(ROOT, "tests", "cpp", "kernels_match_reference")


def test_host_mirror_compiles_as_cpp17():
    cmd = ["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(ROOT, 'staleynet_amd', 'host')}", SOURCE]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr


@pytest.mark.gpu
def test_reference_sweep_through_the_cpp_mirror():
    assert os.path.exists(BINARY), "build the C++ tests first (__graft_entry__.build())"
    proc = subprocess.run([BINARY], capture_output=True, text=True, timeout=300)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "183 of 183 cases passed" in proc.stdout
