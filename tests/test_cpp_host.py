"""The C++ host mirror (include/deltanet.hpp) through its own test binary,
tests/cpp/test_host.cpp: argument checks on the CPU, values against the
oracle on the GPU. The binary is built by __graft_entry__.build()
(make -C tests/cpp)."""

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BIN = ROOT / "tests" / "cpp" / "_build" / "test_host"


def run_binary(mode, timeout):
    if not BIN.exists():
        # Host code only (g++), seconds: build it against the built libraries.
        subprocess.run(["make", "-C", str(ROOT / "tests" / "cpp")], check=True,
                       capture_output=True, timeout=300)
    r = subprocess.run([str(BIN), mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "all passed" in r.stdout


def test_cpp_host_argument_checks():
    run_binary("--host-only", 60)


@pytest.mark.gpu
def test_cpp_host_values_on_gpu():
    run_binary("--gpu", 120)
