"""Builds the gfx950 GEMM library in-tree: ``staleynet_amd/libstaleynet_gemm.so``.

Every source under ``csrc/`` is compiled by ``hipcc --offload-arch=gfx950``
(device code for MI355X only) and linked into one shared library whose C ABI
is ``include/staleynet_gemm.h``. Objects go to ``staleynet_amd/_build/``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PACKAGE_DIR)
CSRC = os.path.join(PACKAGE_DIR, "csrc")
BUILD_DIR = os.path.join(PACKAGE_DIR, "_build")
LIBRARY = os.path.join(PACKAGE_DIR, "libstaleynet_gemm.so")
INCLUDE = os.path.join(REPO_ROOT, "include")

SOURCES = ["context.cpp", "gemm_mfma.hip", "gemm_dma.hip", "gemm_bf16.hip", "gemm_simple.hip", "gemv.hip", "bias.hip",
           "softmax.hip", "loss.hip", "heads.hip", "attention.hip", "bf16_stage.hip",
           "synth.hip", "route.hip", "noalloc.hip", "attention_backward.hip",
           "gemm_bf16_wide.hip"]

# Packed-fp32 instructions are switched off: some of their forms have given
# wrong results on these machines, and the kernels here never need them.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise FileNotFoundError("hipcc not found (ROCm is required to build the GEMM library)")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "is not a recognized feature for this target"
    lines = [ln for ln in proc.stdout.splitlines() if noise not in ln]
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n" + "\n".join(lines))
    if lines:
        print("\n".join(lines))


def build(jobs: int = 8) -> str:
    """Compiles every source and links the library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    cc = hipcc()
    objects = []
    commands = []
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        objects.append(obj)
        commands.append([cc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(commands)))) as pool:
        list(pool.map(_run, commands))
    tmp = LIBRARY + ".tmp"
    _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objects])
    os.replace(tmp, LIBRARY)
    return LIBRARY


def build_oracle() -> str:
    """Builds the CPU oracle (test infrastructure) with its Makefile."""
    oracle_dir = os.path.join(REPO_ROOT, "oracle")
    _run(["make", "-s", "-C", oracle_dir, "-B", "liboracle.so"])
    return os.path.join(oracle_dir, "liboracle.so")


CPP_TESTS = ["kernels_match_reference"]


def build_cpp_tests() -> list[str]:
    """Builds the C++ parity tests (tests/cpp) against the library, the C++
    host mirror (host/staleynet_cuda.hpp) and the oracle. Run from the tests."""
    tests_dir = os.path.join(REPO_ROOT, "tests", "cpp")
    oracle_dir = os.path.join(REPO_ROOT, "oracle")
    outputs = []
    for name in CPP_TESTS:
        out = os.path.join(tests_dir, name)
        _run(["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", f"-I{INCLUDE}", f"-I{os.path.join(PACKAGE_DIR, 'host')}",
              os.path.join(tests_dir, name + ".cpp"), "-o", out,
              f"-L{PACKAGE_DIR}", "-lstaleynet_gemm", f"-L{oracle_dir}", "-loracle",
              "-L/opt/rocm/lib", "-Wl,-rpath-link,/opt/rocm/lib",
              "-Wl,-rpath,$ORIGIN/../../staleynet_amd:$ORIGIN/../../oracle"])
        outputs.append(out)
    return outputs


if __name__ == "__main__":
    print(build())
    print(build_oracle())
    print(build_cpp_tests())
