"""The element encoders of the gfx950 quantize kernels (jalapenos-at-home_amd/
csrc/mx_encode.h, compiled for the device by quant.hip and for the host here)
against the oracle's quantizers on every magnitude an MX block can hold after
division by its scale: every float in [0, 8) for E2M1 (python/quantize_mxfp4.py:
18-39 restated: searchsorted over the midpoints, ties to the even code,
saturation above 5) and every float in [0, 512) for E4M3 (nearest, ties to
even, saturation at 448). The kernels' bit-level forms -- the mantissa rounded
to 1 or 3 bits, half to even, and rint below the normal range -- must give the
same code for every one of them."""
import subprocess
from pathlib import Path

CPP = Path(__file__).resolve().parent / "cpp"


def test_element_encoders_match_oracle_on_every_float():
    from oracle import mx4_oracle

    if not mx4_oracle.LIB_PATH.exists():
        mx4_oracle.build()
    subprocess.run(["make", "-C", str(CPP), "--no-print-directory", "mx_encode_exhaustive"], check=True,
                   capture_output=True)
    r = subprocess.run([str(CPP / "mx_encode_exhaustive")], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "E2M1 [0, 8): checked 1090519040 values, 0 mismatches" in r.stdout
    assert "E4M3 [0, 512): checked 1140850688 values, 0 mismatches" in r.stdout
