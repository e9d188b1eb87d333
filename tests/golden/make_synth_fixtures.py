"""Writes tests/golden/synth_fixtures.json from the oracle's generator.

The reference defines no input generator, so this build defines one (SplitMix64 ->
Box-Muller in fp64 -> x sigma -> f32 -> bf16, all round-to-nearest-even). These
fixtures freeze its first values and the SHA-256 of the single-GEMV workload
(W [6144, 2048] bf16 N(0, 0.02) from seed 0, quantized; x bf16 [1, 2048] N(0, 1)
from seed 1) so that every implementation of the generator -- host or device --
is checked against the same bits. Run: python tests/golden/make_synth_fixtures.py
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import mx4_oracle as o  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main() -> None:
    out = {"about": __doc__.strip().splitlines()[0], "prefixes": {}}
    for seed, sigma in [(0, 0.02), (1, 1.0), (2, 0.02)]:
        out["prefixes"][f"seed{seed}_sigma{sigma}"] = {
            "seed": seed, "sigma": sigma,
            "bf16": o.synth_bf16(seed, sigma, 64).tolist(),
        }
    n, k = 6144, 2048
    wbits = o.synth_bf16(0, 0.02, n * k)
    packed, scales = o.quantize(o.bf16_to_f32(wbits).reshape(n, k))
    xbits = o.synth_bf16(1, 1.0, k)
    x = o.bf16_to_f32(xbits).reshape(1, k)
    y = o.matmul(x, packed, scales)
    out["gemv_2048x6144"] = {
        "w_seed": 0, "w_sigma": 0.02, "x_seed": 1, "x_sigma": 1.0, "n": n, "k": k,
        "sha256_w_bf16": sha(wbits), "sha256_packed": sha(packed), "sha256_scales": sha(scales),
        "sha256_x_bf16": sha(xbits), "sha256_y_f32": sha(y),
        "y_first8": [float(v) for v in y[0, :8]],
        "argmax": o.argmax(y[0]),
    }
    path = Path(__file__).resolve().parent / "synth_fixtures.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(path)


if __name__ == "__main__":
    main()
