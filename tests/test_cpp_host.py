"""The C++ host layer (jalapenos-at-home_amd/host/engine.hpp) and its tests
(tests/cpp/test_engine.cpp), which restate the reference's own tests for this
path (tests/mxfp4.rs, engine/src/mxfp4.rs:56-65, engine/src/metal.rs:86-114)
against the C++ mirror of the reference's types."""
import subprocess
from pathlib import Path

import pytest

CPP = Path(__file__).resolve().parent / "cpp"
BIN = CPP / "test_engine"


def _run(*args):
    r = subprocess.run([str(BIN), *args], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    return r


def test_cpp_host_logic():
    """Storage validation with the reference's messages and the C ABI's validate: no device."""
    subprocess.run(["make", "-C", str(CPP), "--no-print-directory"], check=True, capture_output=True)
    r = _run("--cpu-only")
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failed" in r.stdout


@pytest.mark.gpu
def test_cpp_host_on_device():
    """Every C++ test, the device ones included, through libmx4hip.so."""
    assert BIN.exists(), "tests/cpp/test_engine is built by __graft_entry__.build()"
    r = _run()
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failed" in r.stdout
