"""ctypes binding of libmx4hip.so (include/mx4.h) for tests and the benchmark.

The library is the product: every call here goes straight to the HIP kernels
through the C ABI. There is no CPU fallback -- if the library is missing or no
gfx950 device is present the calls raise.
"""
from __future__ import annotations

import ctypes
import re
import weakref
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmx4hip.so"
HEADER = HERE.parent / "include" / "mx4.h"

MX4_OK = 0
STATUS = {
    0: "MX4_OK", 1: "MX4_ERR_ARGUMENT", 2: "MX4_ERR_SHAPE", 3: "MX4_ERR_TOO_LARGE",
    4: "MX4_ERR_LENGTH", 5: "MX4_ERR_NAN_SCALE", 6: "MX4_ERR_NON_FINITE",
    7: "MX4_ERR_DEVICE", 8: "MX4_ERR_NO_MEMORY", 9: "MX4_ERR_UNSUPPORTED",
}
ERR_TOO_LARGE = 3
ERR_UNSUPPORTED = 9
F32, BF16 = 0, 1
PATH_AUTO, PATH_GEMV, PATH_SKINNY, PATH_GENERIC, PATH_PREFILL, PATH_GEMM = 0, 1, 2, 3, 4, 5
ACT_MXFP4, ACT_MXFP8 = 1, 2

_vp = ctypes.c_void_p
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_int = ctypes.c_int

SIGNATURES = {
    "qwen_hip_create": (_vp, []),
    "qwen_hip_destroy": (None, [_vp]),
    "qwen_hip_matmul": (ctypes.c_bool, [_vp, _f32p, _vp, _u8p, _f32p, _u32, _u32, _u32]),
    "qwen_hip_set_cache_limit": (None, [_vp, _u64]),
    "mx4_create": (_int, [_int, ctypes.POINTER(_vp)]),
    "mx4_destroy": (None, [_vp]),
    "mx4_last_error": (ctypes.c_char_p, []),
    "mx4_device_count": (_int, []),
    "mx4_compute_units": (_int, [_vp, ctypes.POINTER(_int)]),
    "mx4_set_stream": (_int, [_vp, _vp]),
    "mx4_get_stream": (_vp, [_vp]),
    "mx4_synchronize": (_int, [_vp]),
    "mx4_validate": (_int, [_u64, _u64, _u64, _u8p, _u64]),
    "mx4_malloc": (_int, [_vp, _u64, ctypes.POINTER(_vp)]),
    "mx4_free": (_int, [_vp, _vp]),
    "mx4_upload": (_int, [_vp, _vp, _vp, _u64]),
    "mx4_download": (_int, [_vp, _vp, _vp, _u64]),
    "mx4_copy": (_int, [_vp, _vp, _vp, _u64]),
    "mx4_weight_upload": (_int, [_vp, _u8p, _u8p, _u32, _u32, ctypes.POINTER(_vp)]),
    "mx4_weight_wrap": (_int, [_vp, _vp, _vp, _u32, _u32, ctypes.POINTER(_vp)]),
    "mx4_weight_release": (None, [_vp]),
    "mx4_weight_info": (_int, [_vp, ctypes.POINTER(_u32), ctypes.POINTER(_u32),
                               ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "mx4_matmul": (_int, [_vp, _vp, _int, _u32, _vp, _vp]),
    "mx4_matmul_path": (_int, [_vp, _vp, _int, _u32, _vp, _vp, _int]),
    "mx4_matmul_prefill": (_int, [_vp, _vp, _int, _u32, _vp, _int, _vp]),
    "mx4_matmul_prefill_noalloc": (_int, [_vp, _vp, _int, _u32, _vp, _int, _vp]),
    "mx4_matmul_group": (_int, [_vp, _vp, _int, _u32, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _u32]),
    "mx4_gemv_config": (_int, [_vp, _vp, _int, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _u32, _int, _int, _int, _u32]),
    "mx4_gemv_tokens_config": (_int, [_vp, _vp, _u32, _vp, _vp, _u32, _u32]),
    "mx4_gemm_config": (_int, [_vp, _vp, _int, _u32, _vp, _vp, _int, _int, _int, _int, _int]),
    "mx4_weight_footprint": (_int, [_vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "mx4_weight_release_prefill": (_int, [_vp]),
    "mx4_weight_drop_stored": (_int, [_vp]),
    "mx4_matmul_batch": (_int, [_vp, _vp, _u32]),
    "mx4_matmul_mx": (_int, [_vp, _vp, _vp, _int, _u32, _vp, _vp]),
    "mx4_reserve_prefill": (_int, [_vp, _u32, _u32]),
    "mx4_weight_prepare_prefill": (_int, [_vp]),
    "mx4_matmul_argmax": (_int, [_vp, _vp, _int, _vp, _vp, _vp]),
    "mx4_embed": (_int, [_vp, _vp, _vp, _u32, _vp]),
    "mx4_weight_upload_bf16": (_int, [_vp, _vp, _u32, _u32, ctypes.POINTER(_vp)]),
    "mx4_prefill_act_bytes": (_int, [_u32, _u32, _int, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "mx4_prefill_quantize": (_int, [_vp, _vp, _int, _u32, _u32, _int, _vp, _vp]),
    "mx4_prefill_matmul": (_int, [_vp, _vp, _vp, _int, _u32, _vp, _vp]),
    "mx4_prefill_config": (_int, [_vp, _vp, _vp, _int, _u32, _vp, _vp, _u32, _u32, _u32]),
    "mx4_prefill_matmul_group": (_int, [_vp, _vp, _vp, _int, _u32, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _u32]),
    "mx4_prefill_group_config": (_int, [_vp, _vp, _vp, _int, _u32, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _u32,
                                        _u32, _u32, _u32]),
    "mx4_matmul_prefill_group": (_int, [_vp, _vp, _int, _u32, ctypes.POINTER(_vp), _int, ctypes.POINTER(_vp), _u32]),
    "mx4_pass_begin": (_int, [_vp]),
    "mx4_pass_end": (_int, [_vp, ctypes.POINTER(_vp)]),
    "mx4_pass_launch": (_int, [_vp, _vp]),
    "mx4_pass_release": (None, [_vp]),
    "mx4_dequantize": (_int, [_vp, _vp, _vp]),
    "mx4_quantize": (_int, [_vp, _vp, _int, _u64, _u32, _vp, _vp]),
    "mx4_quantize_fp8": (_int, [_vp, _vp, _int, _u64, _u32, _vp, _vp]),
    "mx4_argmax_rows": (_int, [_vp, _vp, _u32, _u32, _vp]),
    "mx4_synth_bf16": (_int, [_vp, _u64, ctypes.c_double, _u64, _u64, _vp]),
    "mx4_synth_weight": (_int, [_vp, _u64, ctypes.c_double, _u32, _u32, _vp, _vp]),
    "mx4_timer_begin": (_int, [_vp]),
    "mx4_timer_end": (_int, [_vp, ctypes.POINTER(ctypes.c_double)]),
    "mx4_decode_table": (_int, [_vp, _int, _vp]),
    "mx4_mfma_ceiling": (_int, [_vp, _int, _int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
}


def _handles(ws) -> "ctypes.Array":
    return (_vp * len(ws))(*[w.handle for w in ws])


def _ptrs(bufs) -> "ctypes.Array":
    return (_vp * len(bufs))(*[b.ptr for b in bufs])


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b((?:qwen_hip|mx4)_[a-z0-9_]+)\s*\(", text)))


class Op(ctypes.Structure):
    """mx4_op: one projection of a batch or recorded pass."""
    _fields_ = [("x", _vp), ("y", _vp), ("w", _vp), ("m", _u32), ("x_type", ctypes.c_int32)]


class Mx4Error(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def last_error() -> str:
    return lib().mx4_last_error().decode()


def check(status: int) -> None:
    if status != MX4_OK:
        raise Mx4Error(status, last_error())


def device_count() -> int:
    return lib().mx4_device_count()


def validate(shape, packed: np.ndarray, scales: np.ndarray) -> int:
    """Host-only check (engine/src/mxfp4.rs:11-25); returns the status code."""
    rows, cols = shape
    scales = np.ascontiguousarray(scales, dtype=np.uint8).reshape(-1)
    return lib().mx4_validate(rows, cols, packed.size, scales.ctypes.data_as(_u8p), scales.size)


def _ptr(a: np.ndarray, ty=_vp):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ty)


class DeviceBuffer:
    """Device allocation owned by a Context (hipMalloc through the C ABI)."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = _vp()
        check(lib().mx4_malloc(ctx.handle, max(self.nbytes, 1), ctypes.byref(p)))
        self.ptr = p.value

    def upload(self, a: np.ndarray, offset: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().mx4_upload(self.ctx.handle, self.ptr + offset, _ptr(a), a.nbytes))
        return self

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        check(lib().mx4_download(self.ctx.handle, _ptr(out), self.ptr + offset, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib().mx4_free(self.ctx.handle, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.ctx.handle:
                lib().mx4_free(self.ctx.handle, self.ptr)
        except Exception:
            pass


class Weight:
    """A resident MXFP4 weight (engine/src/gpu.rs:225-237)."""

    def __init__(self, ctx: "Context", handle: int, rows: int, cols: int, keep=None):
        self.ctx, self.handle, self.rows, self.cols = ctx, handle, rows, cols
        self._keep = keep

    @property
    def nbytes(self) -> int:
        return self.rows * self.cols // 2 + self.rows * self.cols // 32

    def prepare_prefill(self) -> None:
        """Build the matrix-core operand copy now (needed before recording prefill into a pass)."""
        check(lib().mx4_weight_prepare_prefill(self.handle))

    def footprint(self) -> "tuple[int, int]":
        """HBM bytes of the stored layout and of the matrix-core copy."""
        a, b = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().mx4_weight_footprint(self.handle, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def release_prefill(self) -> None:
        check(lib().mx4_weight_release_prefill(self.handle))

    def drop_stored(self) -> None:
        check(lib().mx4_weight_drop_stored(self.handle))

    def release(self) -> None:
        # after mx4_destroy of its context the handle is detached (its device
        # memory already freed) and releasing it only deletes the handle
        if self.handle:
            lib().mx4_weight_release(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Context:
    def __init__(self, device: int = 0):
        h = _vp()
        check(lib().mx4_create(device, ctypes.byref(h)))
        self.handle = h.value
        self._weights: "weakref.WeakSet[Weight]" = weakref.WeakSet()

    def close(self) -> None:
        if self.handle:
            for w in list(self._weights):
                w.release()
            lib().mx4_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # memory
    def buffer(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        return DeviceBuffer(self, a.nbytes).upload(a)

    def synchronize(self) -> None:
        check(lib().mx4_synchronize(self.handle))

    # weights
    def upload_weight(self, packed: np.ndarray, scales: np.ndarray, rows: int, cols: int) -> Weight:
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        h = _vp()
        check(lib().mx4_weight_upload(self.handle, _ptr(packed, _u8p), _ptr(scales, _u8p), rows, cols,
                                      ctypes.byref(h)))
        return self._track(Weight(self, h.value, rows, cols))

    def upload_weight_bf16(self, bits: np.ndarray, rows: int, cols: int) -> Weight:
        """Tensor::bf16: bf16 bit patterns [rows][cols], resident in HBM."""
        bits = np.ascontiguousarray(bits, dtype=np.uint16)
        h = _vp()
        check(lib().mx4_weight_upload_bf16(self.handle, _ptr(bits, _u16p), rows, cols, ctypes.byref(h)))
        return self._track(Weight(self, h.value, rows, cols))

    def _track(self, w: Weight) -> Weight:
        self._weights.add(w)
        return w

    def wrap_weight(self, packed: DeviceBuffer, scales: DeviceBuffer, rows: int, cols: int,
                    packed_offset: int = 0, scales_offset: int = 0) -> Weight:
        h = _vp()
        check(lib().mx4_weight_wrap(self.handle, packed.ptr + packed_offset, scales.ptr + scales_offset,
                                    rows, cols, ctypes.byref(h)))
        return self._track(Weight(self, h.value, rows, cols, keep=(packed, scales)))

    def synth_weight(self, seed: int, rows: int, cols: int, sigma: float = 0.02) -> Weight:
        """The weight recipe generated in HBM (no host copy)."""
        pb = rows * cols // 2
        soff = (pb + 255) // 256 * 256
        buf = self.buffer(soff + rows * cols // 32)
        check(lib().mx4_synth_weight(self.handle, seed, sigma, rows, cols, buf.ptr, buf.ptr + soff))
        return self.wrap_weight(buf, buf, rows, cols, 0, soff)

    def weight_device_arrays(self, w: Weight):
        packed = _vp()
        scales = _vp()
        check(lib().mx4_weight_info(w.handle, None, None, ctypes.byref(packed), ctypes.byref(scales)))
        return packed.value, scales.value

    def download_weight(self, w: Weight):
        p, s = self.weight_device_arrays(w)
        packed = np.empty((w.rows, w.cols // 2), dtype=np.uint8)
        scales = np.empty((w.rows, w.cols // 32), dtype=np.uint8)
        check(lib().mx4_download(self.handle, _ptr(packed), p, packed.nbytes))
        check(lib().mx4_download(self.handle, _ptr(scales), s, scales.nbytes))
        return packed, scales

    # compute (asynchronous on the context stream)
    def matmul(self, x: DeviceBuffer, xtype: int, m: int, w: Weight, y: DeviceBuffer,
               path: int = PATH_AUTO) -> None:
        check(lib().mx4_matmul_path(self.handle, x.ptr, xtype, m, w.handle, y.ptr, path))

    def matmul_ptr(self, xptr: int, xtype: int, m: int, w: Weight, yptr: int, path: int = PATH_AUTO) -> None:
        check(lib().mx4_matmul_path(self.handle, xptr, xtype, m, w.handle, yptr, path))

    def matmul_group(self, xptr: int, xtype: int, m: int, ws, yptrs) -> None:
        n = len(ws)
        wa = (_vp * n)(*[w.handle for w in ws])
        ya = (_vp * n)(*yptrs)
        check(lib().mx4_matmul_group(self.handle, xptr, xtype, m, wa, ya, n))

    def gemv_config(self, xptr: int, xtype: int, ws, yptrs, team: int = 0, rows: int = 0,
                    teams: int = 0, tpw: int = 0) -> None:
        """M = 1 GEMV with an explicit configuration: waves per team, rows per team,
        number of teams, teams per workgroup (0 keeps a default)."""
        if isinstance(ws, Weight):
            ws, yptrs = [ws], [yptrs]
        n = len(ws)
        wa = (_vp * n)(*[w.handle for w in ws])
        ya = (_vp * n)(*yptrs)
        check(lib().mx4_gemv_config(self.handle, xptr, xtype, wa, ya, n, team, rows, tpw, teams))

    def matmul_prefill(self, x: DeviceBuffer, xtype: int, m: int, w: Weight, act: int, y: DeviceBuffer) -> None:
        check(lib().mx4_matmul_prefill(self.handle, x.ptr, xtype, m, w.handle, act, y.ptr))

    def matmul_prefill_noalloc(self, x: DeviceBuffer, xtype: int, m: int, w: Weight, act: int,
                               y: DeviceBuffer) -> None:
        """mx4_matmul_prefill with the library's fixed per-device workspace (allocates nothing)."""
        check(lib().mx4_matmul_prefill_noalloc(self.handle, x.ptr, xtype, m, w.handle, act, y.ptr))

    def matmul_prefill_group(self, x: DeviceBuffer, xtype: int, m: int, ws, act: int, ys) -> None:
        """Requantize x once, then one block-scaled MFMA launch for 1..4 weights (ys: DeviceBuffers)."""
        wa, ya = _handles(ws), _ptrs(ys)
        check(lib().mx4_matmul_prefill_group(self.handle, x.ptr, xtype, m, wa, act, ya, len(ws)))

    def make_ops(self, ops) -> "ctypes.Array[Op]":
        """ops: iterable of (x_ptr, x_type, m, Weight, y_ptr)."""
        ops = list(ops)
        arr = (Op * len(ops))()
        for i, (xp, xt, m, w, yp) in enumerate(ops):
            arr[i] = Op(xp, yp, w.handle, m, xt)
        return arr

    def matmul_batch(self, ops_array) -> None:
        check(lib().mx4_matmul_batch(self.handle, ops_array, len(ops_array)))

    def record(self, fn) -> "Pass":
        """Record everything fn() enqueues into a replayable pass (HIP graph)."""
        check(lib().mx4_pass_begin(self.handle))
        try:
            fn()
        except BaseException:
            # end the capture and drop what was recorded
            h = _vp()
            if lib().mx4_pass_end(self.handle, ctypes.byref(h)) == 0 and h.value:
                lib().mx4_pass_release(h.value)
            raise
        h = _vp()
        check(lib().mx4_pass_end(self.handle, ctypes.byref(h)))
        return Pass(self, h.value)

    def reserve_prefill(self, max_m: int, max_cols: int) -> None:
        check(lib().mx4_reserve_prefill(self.handle, max_m, max_cols))

    def matmul_mx(self, xq: DeviceBuffer, xs: DeviceBuffer, act: int, m: int, w: Weight, y: DeviceBuffer) -> None:
        check(lib().mx4_matmul_mx(self.handle, xq.ptr, xs.ptr, act, m, w.handle, y.ptr))

    def prefill_act_buffers(self, m: int, cols: int, act: int) -> "tuple[DeviceBuffer, DeviceBuffer]":
        """Device buffers for activations requantized in the matrix-core layout."""
        cb, sb = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().mx4_prefill_act_bytes(m, cols, act, ctypes.byref(cb), ctypes.byref(sb)))
        return self.buffer(cb.value), self.buffer(sb.value)

    def prefill_quantize(self, x: DeviceBuffer, xtype: int, m: int, cols: int, act: int, codes: DeviceBuffer,
                         scales: DeviceBuffer) -> None:
        check(lib().mx4_prefill_quantize(self.handle, x.ptr, xtype, m, cols, act, codes.ptr, scales.ptr))

    def prefill_matmul(self, codes: DeviceBuffer, scales: DeviceBuffer, act: int, m: int, w: Weight,
                       y: DeviceBuffer) -> None:
        check(lib().mx4_prefill_matmul(self.handle, codes.ptr, scales.ptr, act, m, w.handle, y.ptr))

    def prefill_matmul_group(self, codes: DeviceBuffer, scales: DeviceBuffer, act: int, m: int, ws, ys) -> None:
        """mx4_prefill_matmul over 1..4 weights of the same K in one launch (ys: DeviceBuffers)."""
        wa, ya = _handles(ws), _ptrs(ys)
        check(lib().mx4_prefill_matmul_group(self.handle, codes.ptr, scales.ptr, act, m, wa, ya, len(ws)))

    def prefill_group_config(self, codes: DeviceBuffer, scales: DeviceBuffer, act: int, m: int, ws, ys,
                             tile_m: int, tile_n: int, split_k: int) -> int:
        """Grouped prefill GEMM with an explicit instance; returns the status."""
        wa, ya = _handles(ws), _ptrs(ys)
        return lib().mx4_prefill_group_config(self.handle, codes.ptr, scales.ptr, act, m, wa, ya, len(ws),
                                              tile_m, tile_n, split_k)

    def gemm_config(self, x: DeviceBuffer, xtype: int, m: int, w: Weight, y: DeviceBuffer, wm: int, wn: int,
                    tm: int, tn: int, ks: int = 0) -> int:
        """Exact tiled GEMM with an explicit instance and K split; returns the status (MX4_ERR_UNSUPPORTED if none)."""
        return lib().mx4_gemm_config(self.handle, x.ptr, xtype, m, w.handle, y.ptr, wm, wn, tm, tn, ks)

    def gemv_tokens_config(self, x: DeviceBuffer, m: int, w: Weight, y: DeviceBuffer, teams: int, tpw: int) -> int:
        """Few-token GEMV (bf16 x) with an explicit launch shape; returns the status."""
        return lib().mx4_gemv_tokens_config(self.handle, x.ptr, m, w.handle, y.ptr, teams, tpw)

    def prefill_config(self, codes: DeviceBuffer, scales: DeviceBuffer, act: int, m: int, w: Weight,
                       y: DeviceBuffer, tile_m: int, tile_n: int, split_k: int) -> int:
        """Prefill GEMM with an explicit instance; returns the status (MX4_ERR_UNSUPPORTED if none)."""
        return lib().mx4_prefill_config(self.handle, codes.ptr, scales.ptr, act, m, w.handle, y.ptr,
                                        tile_m, tile_n, split_k)

    def matmul_argmax(self, x: DeviceBuffer, xtype: int, w: Weight, y, idx: DeviceBuffer) -> None:
        """M = 1 projection + greedy argmax into idx (uint32); y: DeviceBuffer or None."""
        check(lib().mx4_matmul_argmax(self.handle, x.ptr, xtype, w.handle, y.ptr if y is not None else None, idx.ptr))

    def embed(self, w: Weight, ids: DeviceBuffer, count: int, out: DeviceBuffer) -> None:
        check(lib().mx4_embed(self.handle, w.handle, ids.ptr, count, out.ptr))

    def dequantize(self, w: Weight, out: DeviceBuffer) -> None:
        check(lib().mx4_dequantize(self.handle, w.handle, out.ptr))

    def quantize(self, x: DeviceBuffer, xtype: int, rows: int, cols: int, packed: DeviceBuffer,
                 scales: DeviceBuffer) -> None:
        check(lib().mx4_quantize(self.handle, x.ptr, xtype, rows, cols, packed.ptr, scales.ptr))

    def quantize_fp8(self, x: DeviceBuffer, xtype: int, rows: int, cols: int, codes: DeviceBuffer,
                     scales: DeviceBuffer) -> None:
        check(lib().mx4_quantize_fp8(self.handle, x.ptr, xtype, rows, cols, codes.ptr, scales.ptr))

    def argmax_rows(self, x: DeviceBuffer, rows: int, width: int, out: DeviceBuffer) -> None:
        check(lib().mx4_argmax_rows(self.handle, x.ptr, rows, width, out.ptr))

    def synth_bf16(self, seed: int, sigma: float, count: int, out: DeviceBuffer, start: int = 0) -> None:
        check(lib().mx4_synth_bf16(self.handle, seed, sigma, start, count, out.ptr))

    def decode_table(self, mode: int) -> np.ndarray:
        out = self.buffer(256 * 16 * 4)
        check(lib().mx4_decode_table(self.handle, mode, out.ptr))
        return out.download(np.float32).reshape(256, 16)

    def compute_units(self) -> int:
        n = ctypes.c_int()
        check(lib().mx4_compute_units(self.handle, ctypes.byref(n)))
        return n.value

    def mfma_ceiling(self, shape: int, random_codes: bool) -> "tuple[float, float]":
        """Matrix-core ceiling probe: (PFLOP/s, median shader clock in GHz) of
        back-to-back MFMAs (shape 0: scaled FP4 32x32x64, 1: scaled FP4
        16x16x128, 2: scaled FP8 x FP4 32x32x64, 3: bf16 32x32x16)."""
        pf, ghz = ctypes.c_double(), ctypes.c_double()
        check(lib().mx4_mfma_ceiling(self.handle, shape, int(random_codes), ctypes.byref(pf), ctypes.byref(ghz)))
        return pf.value, ghz.value

    def timer_begin(self) -> None:
        check(lib().mx4_timer_begin(self.handle))

    def timer_end(self) -> float:
        ms = ctypes.c_double()
        check(lib().mx4_timer_end(self.handle, ctypes.byref(ms)))
        return ms.value


class Pass:
    def __init__(self, ctx: Context, handle: int):
        self.ctx, self.handle = ctx, handle

    def launch(self) -> None:
        check(lib().mx4_pass_launch(self.ctx.handle, self.handle))

    def release(self) -> None:
        if self.handle:
            lib().mx4_pass_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Hip:
    """Per-call backend over qwen_hip_* with the shape of the reference's Metal
    wrapper (engine/src/metal.rs:21-72): construct once, matmul(x, packed,
    scales) -> y, synchronous, raises on failure (the reference asserts)."""

    def __init__(self):
        self.handle = lib().qwen_hip_create()
        if not self.handle:
            raise RuntimeError(f"could not initialize HIP: {last_error()}")

    def matmul(self, x: np.ndarray, w: np.ndarray, scales=None) -> np.ndarray:
        """w: packed MXFP4 bytes with `scales`, or (scales None) bf16 bits [cols][inner]
        -- the two arms of engine/src/metal.rs:40-51. The arrays must stay alive and
        unchanged while cached: the device copies are keyed by their address."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, inner = x.shape
        if scales is None:
            if w.dtype != np.uint16:
                raise TypeError("bf16 weights are uint16 bit patterns")
            cols = w.size // inner
            sp = None
        else:
            cols = w.size * 2 // inner
            sp = _ptr(scales, _u8p)
        y = np.empty((rows, cols), dtype=np.float32)
        ok = lib().qwen_hip_matmul(self.handle, _ptr(x, _f32p), _ptr(w), sp, _ptr(y, _f32p), rows, cols, inner)
        if not ok:
            raise RuntimeError(f"HIP projection failed: {last_error()}")
        return y

    def set_cache_limit(self, nbytes: int) -> None:
        lib().qwen_hip_set_cache_limit(self.handle, nbytes)

    def close(self) -> None:
        if self.handle:
            lib().qwen_hip_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
