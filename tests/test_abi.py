"""The C-ABI library loads, exports every symbol include/mx4.h declares, and its
host-side validation behaves like the reference's (no GPU needed)."""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def mx4():
    import mx4hip

    if not mx4hip.LIB_PATH.exists():
        pytest.fail("libmx4hip.so is not built; run __graft_entry__.build()")
    return mx4hip


def test_library_exports_every_header_symbol(mx4):
    symbols = mx4.header_symbols()
    assert len(symbols) >= 30
    lib = ctypes.CDLL(str(mx4.LIB_PATH))
    missing = [s for s in symbols if not hasattr(lib, s)]
    assert not missing, missing
    # the binding declares exactly the header's functions
    assert sorted(mx4.SIGNATURES) == symbols


def test_every_kernel_launch_stub_is_defined(mx4):
    """Every kernel the host code launches has its launch stub in the library.
    (A device-only builtin that the host pass rejects makes clang drop the
    stubs of the kernels that use it without an error; the library then fails
    to load on a machine with the GPU.)"""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-u", str(mx4.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    missing = [line.split()[-1] for line in out.splitlines() if "device_stub" in line]
    assert not missing, missing[:5]


def test_library_is_built_for_gfx950_only(mx4):
    data = mx4.LIB_PATH.read_bytes()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"sm_"):
        assert other + b"\x00" not in data or other == b"sm_"


def test_validate_matches_reference_rejects(mx4):
    kats = json.loads((GOLDEN / "reference_kats.json").read_text())
    want = {0: mx4.STATUS[2], 1: mx4.STATUS[4], 2: mx4.STATUS[5]}
    for i, case in enumerate(kats["rejects"]["cases"]):  # engine/tests/mxfp4.rs:35-40
        packed = np.zeros(case["packed_len"], np.uint8)
        st = mx4.validate(case["shape"], packed, np.array(case["scales"], np.uint8))
        assert mx4.STATUS[st] == want[i]
    assert "divisible by 32" in mx4.last_error() or "NaN scale" in mx4.last_error()
    assert mx4.validate((1, 32), np.zeros(16, np.uint8), np.array([127], np.uint8)) == 0
    assert mx4.validate((0, 32), np.zeros(0, np.uint8), np.zeros(0, np.uint8)) == 2
    assert mx4.validate((2, 64), np.zeros(64, np.uint8), np.full(4, 254, np.uint8)) == 0


def test_validate_agrees_with_oracle_on_random_cases(mx4, oracle):
    rng = np.random.default_rng(0)
    for _ in range(200):
        rows = int(rng.integers(0, 4))
        cols = int(rng.choice([0, 16, 31, 32, 64, 96]))
        plen = rows * cols // 2 + int(rng.choice([0, 0, -1, 1]))
        slen = max(rows * cols // 32 + int(rng.choice([0, 0, 1])), 0)
        scales = rng.integers(250, 256, max(slen, 1), dtype=np.uint8)[:slen]
        packed = np.zeros(max(plen, 0), np.uint8)
        a = mx4.validate((rows, cols), packed, scales)
        b = oracle.mx_validate((rows, cols), packed, scales)
        # oracle codes: 0 ok, 1 shape, 2 too large, 3 lengths, 4 NaN scale
        assert {0: 0, 1: 2, 2: 3, 3: 4, 4: 5}[b] == a, (rows, cols, plen, slen)


def test_no_device_fails_cleanly(mx4):
    if mx4.device_count() > 0:
        pytest.skip("a GPU is present")
    assert mx4.lib().qwen_hip_create() is None
    with pytest.raises(mx4.Mx4Error):
        mx4.Context()
