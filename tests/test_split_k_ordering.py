"""The split-K arrival protocol of the skinny kernel orders its partial tiles
with agent-scope release/acquire fences (HIP memory model), not with cache
bits and wait counts alone. This CPU test compiles csrc/skinny.hip for gfx950
to assembly and checks every split-K instance (template argument KS > 1):
the release (an L2 write-back, `buffer_wbl2 sc1`, then `s_waitcnt vmcnt(0)`)
comes before the arrival count's atomic add, and the acquire (an L2
invalidate, `buffer_inv sc1`) after it and before the partials are loaded.
The unsplit instances carry neither."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "jalapenos-at-home_amd"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def skinny_asm(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "skinny.s"
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{PKG / 'csrc'}", "-mllvm",
           "-amdgpu-kernarg-preload-count=16", "-S", "--cuda-device-only", str(PKG / "csrc" / "skinny.hip"),
           "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


def kernels(asm):
    """(name, body) of every skinny_kernel instance in the assembly."""
    found = []
    for m in re.finditer(r"^(_Z\S*skinny_kernel\S*):\s*;", asm, re.M):
        start = m.end()
        end = asm.find("s_endpgm", start)
        found.append((m.group(1), asm[start:end]))
    return found


def split_ks(name):
    # template <bool XBF16, int MT, int U, int NU, int TW, bool RESX, int KS,
    # int XLM, int NP>: KS is the integer right after the last bool (RESX)
    m = re.findall(r"Lb[01]ELi(\d+)E", name)
    assert len(m) == 2, name
    return int(m[-1])


def test_split_instances_carry_release_and_acquire(skinny_asm):
    ks = kernels(skinny_asm)
    split = [(n, b) for n, b in ks if split_ks(n) > 1]
    assert len(split) >= 3, "expected the K = 12288 and K = 4096 split-K instances"
    for name, body in split:
        lines = [ln.strip() for ln in body.splitlines() if ln.strip() and not ln.strip().startswith(";")]
        add = [i for i, ln in enumerate(lines) if ln.startswith("global_atomic_add") or ln.startswith("buffer_atomic_add")]
        assert add, f"{name}: no arrival count"
        a = add[0]
        wb = [i for i, ln in enumerate(lines[:a]) if ln.startswith("buffer_wbl2") and "sc1" in ln]
        assert wb, f"{name}: no agent-scope release before the count"
        assert any(ln.startswith("s_waitcnt") and "vmcnt(0)" in ln for ln in lines[wb[-1]:a]), name
        inv = [i for i, ln in enumerate(lines[a:]) if ln.startswith("buffer_inv") and "sc1" in ln]
        assert inv, f"{name}: no agent-scope acquire after the count"
        loads_after = [ln for ln in lines[a + inv[0]:] if ln.startswith("buffer_load_dwordx4")]
        assert loads_after, f"{name}: the partials are not loaded after the acquire"


def test_unsplit_instances_carry_no_fences(skinny_asm):
    for name, body in kernels(skinny_asm):
        if split_ks(name) == 1:
            assert "buffer_wbl2" not in body and "buffer_inv" not in body, name
