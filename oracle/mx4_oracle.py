"""ctypes binding of the CPU oracle (oracle/mx4_oracle.c).

TEST INFRASTRUCTURE ONLY: this is the checker. Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import it. The product path never does.
Every wrapper cites the reference file:line its C function restates.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_mx4.so"

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u64 = ctypes.c_uint64


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    import subprocess

    subprocess.run(["make", "-C", str(HERE), "-B", "--no-print-directory"], check=True)


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
    lib = ctypes.CDLL(str(LIB_PATH))
    sig = {
        "oracle_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "oracle_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
        "oracle_powi2": (ctypes.c_float, [ctypes.c_int32]),
        "oracle_mx_value": (ctypes.c_float, [_u8p, _u8p, _u64]),
        "oracle_mx_values": (None, [_u8p, _u8p, _u64, _u64, _f32p]),
        "oracle_mx_validate": (ctypes.c_int, [_u64, _u64, _u64, _u8p, _u64]),
        "oracle_matmul": (None, [_f32p, _u64, _u64, _u8p, _u8p, _u64, _f32p]),
        "oracle_matmul_bf16": (None, [_f32p, _u64, _u64, _u16p, _u64, _f32p]),
        "oracle_matmul_rows": (None, [_f32p, _u64, _u64, _u8p, _u8p, _u64, _u64, _f32p, ctypes.c_int]),
        "oracle_matmul_f64": (None, [_f32p, _u64, _u64, _u8p, _u8p, _u64, _f64p]),
        "oracle_quantize": (ctypes.c_int, [_f32p, _u64, _u64, _u8p, _u8p]),
        "oracle_dequantize": (None, [_u8p, _u8p, _u64, _u64, _f32p]),
        "oracle_quantize_fp8": (ctypes.c_int, [_f32p, _u64, _u64, _u8p, _u8p]),
        "oracle_fp8_e4m3_value": (ctypes.c_float, [ctypes.c_uint8]),
        "oracle_dequantize_fp8": (None, [_u8p, _u8p, _u64, _u64, _f32p]),
        "oracle_argmax": (_u64, [_f32p, _u64]),
        "oracle_splitmix64": (_u64, [_u64, _u64]),
        "oracle_ln": (ctypes.c_double, [ctypes.c_double]),
        "oracle_cos2pi": (ctypes.c_double, [ctypes.c_double]),
        "oracle_normal": (ctypes.c_double, [_u64, _u64]),
        "oracle_synth_bf16": (None, [_u64, ctypes.c_double, _u64, _u64, _u16p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = _load()
    return _LIB


def _p(a: np.ndarray, ty):
    assert a.flags["C_CONTIGUOUS"], "oracle needs contiguous arrays"
    return a.ctypes.data_as(ty)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """engine/src/lib.rs:74-76 (vectorised: the same shift)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def powi2(e: int) -> float:
    """engine/src/mxfp4.rs:30 (2.0_f32.powi)."""
    return lib().oracle_powi2(e)


def mx_values(packed: np.ndarray, scales: np.ndarray, start: int, end: int) -> np.ndarray:
    """engine/src/mxfp4.rs:35-49."""
    out = np.empty(end - start, dtype=np.float32)
    lib().oracle_mx_values(_p(packed, _u8p), _p(scales, _u8p), start, end, _p(out, _f32p))
    return out


def mx_value(packed: np.ndarray, scales: np.ndarray, index: int) -> float:
    """engine/src/mxfp4.rs:27-33."""
    return lib().oracle_mx_value(_p(packed, _u8p), _p(scales, _u8p), index)


def mx_validate(shape, packed: np.ndarray, scales: np.ndarray) -> int:
    """engine/src/mxfp4.rs:11-25. 0 ok, 1 shape, 2 too large, 3 lengths, 4 NaN scale."""
    rows, cols = shape
    scales = np.ascontiguousarray(scales, dtype=np.uint8).reshape(-1)
    return lib().oracle_mx_validate(rows, cols, packed.size, _p(scales, _u8p), scales.size)


def matmul(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """engine/src/lib.rs:240-266 (MXFP4 arm). x f32 [M,K]; returns f32 [M,N]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    n = packed.size * 2 // k
    out = np.empty((m, n), dtype=np.float32)
    lib().oracle_matmul(_p(x, _f32p), m, k, _p(packed, _u8p), _p(scales, _u8p), n, _p(out, _f32p))
    return out


def matmul_bf16(x: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """engine/src/lib.rs:240-266 (bf16 arm). w_bits u16 [N,K]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    m, k = x.shape
    n = w_bits.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    lib().oracle_matmul_bf16(_p(x, _f32p), m, k, _p(w_bits, _u16p), n, _p(out, _f32p))
    return out


def matmul_rows(x: np.ndarray, packed: np.ndarray, scales: np.ndarray, r0: int, r1: int,
                threads: int = 1) -> np.ndarray:
    """engine/src/lib.rs:240-266 over weight rows [r0, r1) only."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    out = np.empty((m, r1 - r0), dtype=np.float32)
    lib().oracle_matmul_rows(_p(x, _f32p), m, k, _p(packed, _u8p), _p(scales, _u8p), r0, r1,
                             _p(out, _f32p), threads)
    return out


def matmul_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    n = packed.size * 2 // k
    out = np.empty((m, n), dtype=np.float64)
    lib().oracle_matmul_f64(_p(x, _f32p), m, k, _p(packed, _u8p), _p(scales, _u8p), n, _p(out, _f64p))
    return out


def quantize(values: np.ndarray):
    """python/quantize_mxfp4.py:18-39. Raises ValueError like the reference."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    if values.ndim != 2 or values.shape[1] % 32:
        raise ValueError("expected a matrix whose row width is divisible by 32")
    r, c = values.shape
    packed = np.empty((r, c // 2), dtype=np.uint8)
    scales = np.empty((r, c // 32), dtype=np.uint8)
    rc = lib().oracle_quantize(_p(values, _f32p), r, c, _p(packed, _u8p), _p(scales, _u8p))
    if rc == 2:
        raise ValueError("cannot quantize non-finite weights")
    if rc:
        raise ValueError("expected a matrix whose row width is divisible by 32")
    return packed, scales


def dequantize(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """python/quantize_mxfp4.py:42-49."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    r, half = packed.shape
    out = np.empty((r, half * 2), dtype=np.float32)
    lib().oracle_dequantize(_p(packed, _u8p), _p(scales, _u8p), r, half * 2, _p(out, _f32p))
    return out


def quantize_fp8(values: np.ndarray):
    """MX-FP8 (E4M3) activation requant: scale = floor(log2 amax) - 8, RNE, saturate."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    r, c = values.shape
    codes = np.empty((r, c), dtype=np.uint8)
    scales = np.empty((r, c // 32), dtype=np.uint8)
    rc = lib().oracle_quantize_fp8(_p(values, _f32p), r, c, _p(codes, _u8p), _p(scales, _u8p))
    if rc:
        raise ValueError("bad fp8 quantize input")
    return codes, scales


def fp8_value(code: int) -> float:
    return lib().oracle_fp8_e4m3_value(code)


def dequantize_fp8(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    r, c = codes.shape
    out = np.empty((r, c), dtype=np.float32)
    lib().oracle_dequantize_fp8(_p(codes, _u8p), _p(scales, _u8p), r, c, _p(out, _f32p))
    return out


def argmax(values: np.ndarray) -> int:
    """engine/src/model.rs:288-296."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    return int(lib().oracle_argmax(_p(values, _f32p), values.size))


def splitmix64(seed: int, n: int) -> int:
    return int(lib().oracle_splitmix64(seed, n))


def ln(u: float) -> float:
    return lib().oracle_ln(u)


def cos2pi(t: float) -> float:
    return lib().oracle_cos2pi(t)


def normal(seed: int, index: int) -> float:
    return lib().oracle_normal(seed, index)


def synth_bf16(seed: int, sigma: float, count: int, start: int = 0) -> np.ndarray:
    """Synthetic bf16 bits: SplitMix64 -> Box-Muller -> x sigma -> f32 -> bf16."""
    out = np.empty(count, dtype=np.uint16)
    lib().oracle_synth_bf16(seed, sigma, start, count, _p(out, _u16p))
    return out


def synth_weight(seed: int, n: int, k: int, sigma: float = 0.02):
    """Weight recipe: bf16 N(0, sigma) from seed, quantized by the reference rule."""
    bits = synth_bf16(seed, sigma, n * k).reshape(n, k)
    return quantize(bf16_to_f32(bits))


def cpu_cores() -> int:
    return len(os.sched_getaffinity(0))
