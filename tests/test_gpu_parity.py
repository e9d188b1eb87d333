"""GPU parity: the HIP kernels, called through the C ABI, against the CPU oracle.

Bars: bit-exact for decode, quantize, requantize, the generator and argmax.
Matmuls against the oracle r (engine/src/lib.rs:240-266), all three at once:
  * max_i |y_i - r_i| / max_i |r_i| <= 1e-3 (the stated tolerance of the path);
  * the reference's own per-element bound |y - r| < 1e-3 + 1e-5 |r|
    (engine/src/metal.rs:110) on the raw values; only tests whose weights use
    deliberately large scale bytes (outputs of 1e2..1e5) apply it to values
    divided by max |r|, and say so at the call (scaled=True);
  * ||y - r||_2 / ||r||_2 <= 1e-5, the reference's normwise form
    (engine/tests/mxfp4.rs:76-84). Every path here multiplies exactly and sums
    in f32, so only the summation order differs from the oracle (~1e-6).
"""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
KATS = json.loads((GOLDEN / "reference_kats.json").read_text())
REL_TOL = 1e-3

QWEN17 = {"q": (2048, 2048), "k": (1024, 2048), "v": (1024, 2048), "o": (2048, 2048),
          "gate": (6144, 2048), "up": (6144, 2048), "down": (2048, 6144), "lm_head": (151936, 2048)}
QWEN8 = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
         "gate": (12288, 4096), "up": (12288, 4096), "down": (4096, 12288), "lm_head": (151936, 4096)}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def mx4():
    import mx4hip

    if mx4hip.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    return mx4hip


@pytest.fixture(scope="module")
def ctx(mx4):
    c = mx4.Context(0)
    yield c
    c.close()


def f32_bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def max_rel(y, r):
    denom = float(np.max(np.abs(r)))
    return float(np.max(np.abs(y.astype(np.float64) - r.astype(np.float64)))) / (denom if denom else 1.0)


RMS_TOL = 1e-5


def rel_rms(y, r):
    d = y.astype(np.float64) - r.astype(np.float64)
    den = float(np.sqrt(np.sum(r.astype(np.float64) ** 2)))
    return float(np.sqrt(np.sum(d * d))) / (den if den else 1.0)


def assert_close(y, r, what, scaled=False):
    """The three bars of the module docstring. scaled=True divides both sides
    by max |r| before the per-element bound (large-scale test weights only)."""
    y = np.asarray(y, np.float32)
    r = np.asarray(r, np.float32)
    assert y.shape == r.shape, f"{what}: shape {y.shape} != {r.shape}"
    rel = max_rel(y, r)
    assert rel <= REL_TOL, f"{what}: max rel err {rel:.3e}"
    yy, rr = y.astype(np.float64), r.astype(np.float64)
    if scaled:
        s = max(float(np.max(np.abs(rr))), 1.0)
        yy, rr = yy / s, rr / s
    bad = ~(np.abs(yy - rr) < 1e-3 + 1e-5 * np.abs(rr))
    assert not np.any(bad), f"{what}: {int(bad.sum())} elements outside |a-b| < 1e-3 + 1e-5|b|"
    rms = rel_rms(y, r)
    assert rms <= RMS_TOL, f"{what}: relative RMS error {rms:.3e}"
    return rel


def run_matmul(mx4, ctx, x_f32, w, path, xtype=None):
    """Upload x (f32 or its bf16 bits), run one matmul through the C ABI, download y."""
    m, k = x_f32.shape
    xtype = mx4.F32 if xtype is None else xtype
    if xtype == mx4.BF16:
        bits = (f32_bits(x_f32) >> 16).astype(np.uint16)
        assert np.array_equal(f32_bits(x_f32) & 0xFFFF, np.zeros_like(f32_bits(x_f32))), "x not bf16"
        xb = ctx.to_device(bits)
    else:
        xb = ctx.to_device(np.ascontiguousarray(x_f32, np.float32))
    yb = ctx.buffer(m * w.rows * 4)
    ctx.matmul(xb, xtype, m, w, yb, path)
    return yb.download(np.float32).reshape(m, w.rows)


# ------------------------------------------------------------------ decode

def test_decode_table_bit_exact(mx4, ctx, oracle):
    say("decode tables: 16 codes x 255 scale bytes")
    codes = np.arange(16, dtype=np.uint8)
    packed = np.tile((codes[0::2] | (codes[1::2] << 4)).astype(np.uint8), 2 * 255)
    scales = np.arange(255, dtype=np.uint8)
    want = oracle.mx_values(packed, scales, 0, 255 * 32).reshape(255, 32)[:, :16]
    for mode in (0, 1):  # bit construction; hardware converter x 2^(s-127)
        got = ctx.decode_table(mode)[:255]
        bad = np.argwhere(f32_bits(got) != f32_bits(want))
        assert bad.size == 0, f"mode {mode}: first mismatches (s, c) {bad[:8].tolist()}"
    # scale folded into the converter (bf16 and f32 outputs): exact for every
    # scale byte the fast kernels accept (2..252) and up to 254
    for mode in (2, 3):
        got = ctx.decode_table(mode)[2:255]
        bad = np.argwhere(f32_bits(got) != f32_bits(want[2:]))
        assert bad.size == 0, f"mode {mode}: first mismatches (s-2, c) {bad[:8].tolist()}"


def test_dequantize_bit_exact(mx4, ctx, oracle):
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, (37, 96 // 2), dtype=np.uint8)
    scales = rng.integers(0, 255, (37, 96 // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, 37, 96)
    out = ctx.buffer(37 * 96 * 4)
    ctx.dequantize(w, out)
    got = out.download(np.float32)
    want = oracle.mx_values(packed.reshape(-1), scales.reshape(-1), 0, 37 * 96)
    assert np.array_equal(f32_bits(got), f32_bits(want))
    # engine/src/mxfp4.rs:56-65
    w2 = ctx.upload_weight(np.full(16, 0x82, np.uint8), np.zeros(1, np.uint8), 1, 32)
    out2 = ctx.buffer(32 * 4)
    ctx.dequantize(w2, out2)
    v = out2.download(np.float32)
    assert f32_bits(v[0]) == 0x00400000 and f32_bits(v[1]) == 0x80000000


# ------------------------------------------------------------------ quantize

def _quantize_cases(rng):
    return [
        (rng.standard_normal((64, 256)) * 0.02).astype(np.float32),
        (rng.standard_normal((8, 128)) * rng.choice([1e-40, 1e-3, 1, 1e30], (8, 1))).astype(np.float32),
        (rng.integers(-24, 25, (8, 64)) * 0.25).astype(np.float32),   # exact midpoints
        np.where(rng.random((4, 64)) < 0.5, -0.0, 0.0).astype(np.float32),
        np.full((2, 32), 3.0e38, np.float32),
    ]


@pytest.mark.parametrize("xtype", ["f32", "bf16"])
def test_quantize_bit_exact(mx4, ctx, oracle, xtype):
    rng = np.random.default_rng(2)
    for vals in _quantize_cases(rng):
        if xtype == "bf16":
            bits = (f32_bits(vals) >> 16).astype(np.uint16)
            vals = oracle.bf16_to_f32(bits).reshape(vals.shape)
            src = ctx.to_device(bits)
            t = mx4.BF16
        else:
            src = ctx.to_device(vals)
            t = mx4.F32
        r, c = vals.shape
        pk, sc = ctx.buffer(r * c // 2), ctx.buffer(r * c // 32)
        ctx.quantize(src, t, r, c, pk, sc)
        want_p, want_s = oracle.quantize(vals)
        assert np.array_equal(pk.download(np.uint8).reshape(r, -1), want_p)
        assert np.array_equal(sc.download(np.uint8).reshape(r, -1), want_s)


def test_quantize_rejects_non_finite(mx4, ctx):
    vals = np.zeros((1, 32), np.float32)
    vals[0, 3] = np.inf
    src = ctx.to_device(vals)
    pk, sc = ctx.buffer(16), ctx.buffer(1)
    with pytest.raises(mx4.Mx4Error, match="non-finite"):
        ctx.quantize(src, mx4.F32, 1, 32, pk, sc)


def test_quantize_fp8_bit_exact(mx4, ctx, oracle):
    rng = np.random.default_rng(3)
    for vals in _quantize_cases(rng):
        r, c = vals.shape
        src = ctx.to_device(vals)
        cd, sc = ctx.buffer(r * c), ctx.buffer(r * c // 32)
        ctx.quantize_fp8(src, mx4.F32, r, c, cd, sc)
        want_c, want_s = oracle.quantize_fp8(vals)
        assert np.array_equal(cd.download(np.uint8).reshape(r, -1), want_c)
        assert np.array_equal(sc.download(np.uint8).reshape(r, -1), want_s)


# ------------------------------------------------------------------ generator

def test_synth_matches_oracle_generator(mx4, ctx, oracle):
    say("generator: 2M bf16 values")
    n = 1 << 21
    out = ctx.buffer(n * 2)
    for seed, sigma, start in [(0, 0.02, 0), (1, 1.0, 0), (7, 0.02, 12345)]:
        ctx.synth_bf16(seed, sigma, n, out, start=start)
        got = out.download(np.uint16)
        assert np.array_equal(got, oracle.synth_bf16(seed, sigma, n, start=start)), (seed, sigma, start)
    fx = json.loads((GOLDEN / "synth_fixtures.json").read_text())
    for case in fx["prefixes"].values():
        ctx.synth_bf16(case["seed"], case["sigma"], 64, out)
        assert out.download(np.uint16, 64).tolist() == case["bf16"]


def test_synth_weight_matches_recipe(mx4, ctx, oracle):
    import hashlib

    fx = json.loads((GOLDEN / "synth_fixtures.json").read_text())["gemv_2048x6144"]
    w = ctx.synth_weight(fx["w_seed"], fx["n"], fx["k"], fx["w_sigma"])
    packed, scales = ctx.download_weight(w)
    assert hashlib.sha256(packed.tobytes()).hexdigest() == fx["sha256_packed"]
    assert hashlib.sha256(scales.tobytes()).hexdigest() == fx["sha256_scales"]


# ------------------------------------------------------------------ matmul KATs

def test_identity_decodes_every_code(mx4, ctx, oracle):
    kat = KATS["identity_all_codes"]  # engine/tests/mxfp4.rs:9-33
    packed = np.tile(np.array(kat["packed_row"], np.uint8), kat["packed_repeat"])
    w = ctx.upload_weight(packed, np.array(kat["scales"], np.uint8), 1, 32)
    y = run_matmul(mx4, ctx, np.eye(32, dtype=np.float32), w, mx4.PATH_GENERIC)
    # by value, as the reference's assert_eq! on f32 (-0.0 == 0.0) ...
    assert np.array_equal(y.reshape(-1), np.array(kat["expect"], np.float32))
    # ... and bitwise against the oracle, whose 0.0 + (-0.0) sums are +0.0
    want = oracle.matmul(np.eye(32, dtype=np.float32), packed, np.array(kat["scales"], np.uint8))
    assert np.array_equal(f32_bits(y), f32_bits(want))
    # M = 1 one-hot rows through the auto dispatch
    for i in (0, 9, 31):
        x = np.zeros((1, 32), np.float32)
        x[0, i] = 1.0
        y1 = run_matmul(mx4, ctx, x, w, mx4.PATH_AUTO)
        assert y1[0, 0] == np.float32(kat["expect"][i])


def test_rows_and_blocks_use_different_scales(mx4, ctx):
    kat = KATS["rows_and_blocks_use_different_scales"]  # engine/tests/mxfp4.rs:88-105
    w = ctx.upload_weight(np.full(64, kat["packed_fill"], np.uint8), np.array(kat["scales"], np.uint8), 2, 64)
    x = np.zeros(3 * 64, np.float32)
    x[kat["input_ones"]] = 1.0
    y = run_matmul(mx4, ctx, x.reshape(3, 64), w, mx4.PATH_AUTO)
    assert y.reshape(-1).tolist() == kat["expect"]


def test_dropin_matches_cpu_for_decode_and_prefill(mx4, oracle):
    # engine/src/metal.rs:86-114 for the HIP backend through qwen_hip_matmul
    hip = mx4.Hip()
    try:
        packed = (np.arange(21 * 32) % 256).astype(np.uint8)
        scales = (122 + np.arange(21 * 2) % 7).astype(np.uint8)
        for rows in [1, 2, 4, 8, 16, 19, 33]:
            x = (((np.arange(rows * 64) % 37) - 18.0) / 19.0).astype(np.float32).reshape(rows, 64)
            expected = oracle.matmul(x, packed, scales)
            actual = hip.matmul(x, packed, scales)
            assert actual.shape == expected.shape
            assert np.all(np.abs(actual - expected) < 1e-3 + np.abs(expected) * 1e-5), rows
        # the cache is keyed by host pointer: the same arrays are not re-uploaded,
        # a second weight at another address is
        packed2 = packed.copy()
        packed2[:16] = 0x77  # row 0, block 0: all codes 6.0
        x = np.ones((1, 64), np.float32)
        assert not np.array_equal(hip.matmul(x, packed2, scales), hip.matmul(x, packed, scales))
        # failures return false (here: raise), nothing is launched
        with pytest.raises(RuntimeError, match="NaN scale"):
            hip.matmul(x, packed, np.full(42, 255, np.uint8))
    finally:
        hip.close()


def test_dropin_fast_paths_match_cpu(mx4, oracle):
    """qwen_hip_matmul (f32 x from the host, synchronous) on Qwen-width weights,
    where it takes the fast kernels: the M = 1 GEMV, the skinny kernel
    (2..32 rows) and the exact tiled GEMM (33 and more rows), each against the
    oracle with the reference's per-element bound (engine/src/metal.rs:110)."""
    rng = np.random.default_rng(5)
    n, k = 300, 2048
    packed, scales = oracle.synth_weight(17, n, k)
    hip = mx4.Hip()
    try:
        for rows in (1, 3, 16, 33, 70):
            x = (rng.standard_normal((rows, k)) * 0.5).astype(np.float32)
            expected = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
            actual = hip.matmul(x, packed, scales)
            assert actual.shape == expected.shape
            assert_close(actual, expected, f"drop-in rows={rows}")
    finally:
        hip.close()


def test_dropin_bf16_weights_match_cpu(mx4, oracle):
    """engine/src/metal.rs:86-114, the bf16 arm: the decoded quantized weight as
    Tensor::bf16 (scales == NULL), for the same rows, against the reference's
    bf16 matmul (engine/src/lib.rs:255) and within the test's tolerance."""
    hip = mx4.Hip()
    try:
        packed = (np.arange(21 * 32) % 256).astype(np.uint8)
        scales = (122 + np.arange(21 * 2) % 7).astype(np.uint8)
        decoded = oracle.dequantize(packed.reshape(21, 32), scales.reshape(21, 2)).reshape(21, 64)
        bf16 = (f32_bits(decoded) >> 16).astype(np.uint16)
        for rows in [1, 2, 4, 8, 16, 19, 33]:
            x = (((np.arange(rows * 64) % 37) - 18.0) / 19.0).astype(np.float32).reshape(rows, 64)
            expected = oracle.matmul_bf16(x, bf16)
            actual = hip.matmul(x, bf16)
            assert actual.shape == expected.shape
            assert np.all(np.abs(actual - expected) < 1e-3 + np.abs(expected) * 1e-5), rows
            # both arms of the same weight agree (the decode is exact in bf16 here)
            assert np.all(np.abs(actual - hip.matmul(x, packed, scales)) < 1e-3 + np.abs(expected) * 1e-5), rows
    finally:
        hip.close()


@pytest.mark.parametrize("k", [64, 100, 2048])
def test_bf16_weight_resident(mx4, ctx, oracle, k):
    """Tensor::bf16 weights resident in HBM: M in {1, 3, 19, 64}, f32 and bf16
    activations, against the reference's bf16 arm; K = 100 takes the element-wise
    form (rows not 16-byte aligned)."""
    rng = np.random.default_rng(k)
    n = 150
    w_bits = (f32_bits(rng.standard_normal((n, k)).astype(np.float32) * 0.05) >> 16).astype(np.uint16)
    w = ctx.upload_weight_bf16(w_bits, n, k)
    for m in (1, 3, 19, 64):
        xf = rng.standard_normal((m, k)).astype(np.float32)
        xbits = (f32_bits(xf) >> 16).astype(np.uint16)
        xb16 = (xbits.astype(np.uint32) << 16).view(np.float32)
        for xt, host, dev in ((mx4.F32, xf, ctx.to_device(xf)), (mx4.BF16, xb16, ctx.to_device(xbits))):
            yb = ctx.buffer(m * n * 4)
            ctx.matmul(dev, xt, m, w, yb)
            assert_close(yb.download(np.float32).reshape(m, n), oracle.matmul_bf16(host, w_bits), f"bf16 k={k} m={m}")
    with pytest.raises(mx4.Mx4Error, match="MXFP4"):
        ctx.matmul_prefill(ctx.to_device(np.zeros((4, k), np.float32)), mx4.F32, 4, w, mx4.ACT_MXFP4,
                           ctx.buffer(4 * n * 4))


# ------------------------------------------------------------------ GEMV at model shapes

def _sample_rows(n, count, rng):
    if n <= count:
        return np.arange(n)
    return np.unique(np.concatenate([[0, n - 1], rng.choice(n, count, replace=False)]))


@pytest.mark.parametrize("model", ["1.7B", "8B"])
def test_gemv_model_shapes(mx4, ctx, oracle, model):
    shapes = QWEN17 if model == "1.7B" else QWEN8
    rng = np.random.default_rng(4)
    for j, (name, (n, k)) in enumerate(shapes.items()):
        say(f"gemv {model} {name} {k}->{n}")
        w = ctx.synth_weight(100 + j, n, k, 0.02)
        packed, scales = ctx.download_weight(w)
        xbits = oracle.synth_bf16(1, 1.0, k)
        x = oracle.bf16_to_f32(xbits).reshape(1, k)
        rows = _sample_rows(n, 384, rng)
        ref = np.concatenate([oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), int(r), int(r) + 1)
                              for r in rows], axis=1)
        for xtype in (mx4.BF16, mx4.F32):
            y = run_matmul(mx4, ctx, x, w, mx4.PATH_AUTO, xtype)
            assert np.all(np.isfinite(y))
            assert_close(y[:, rows], ref, f"{model} {name} xtype={xtype}")
        w.release()


def test_gemv_6144x2048_against_fixture(mx4, ctx, oracle):
    import hashlib

    fx = json.loads((GOLDEN / "synth_fixtures.json").read_text())["gemv_2048x6144"]
    w = ctx.synth_weight(fx["w_seed"], fx["n"], fx["k"], fx["w_sigma"])
    packed, scales = ctx.download_weight(w)
    x = oracle.bf16_to_f32(oracle.synth_bf16(fx["x_seed"], fx["x_sigma"], fx["k"])).reshape(1, -1)
    ref = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
    assert hashlib.sha256(ref.tobytes()).hexdigest() == fx["sha256_y_f32"]
    for xtype in (mx4.BF16, mx4.F32):
        y = run_matmul(mx4, ctx, x, w, mx4.PATH_GEMV, xtype)
        assert_close(y, ref, "6144 x 2048 GEMV")
        assert oracle.argmax(y[0]) == fx["argmax"]


def test_lm_head_greedy_argmax_identical(mx4, ctx, oracle):
    n, k = QWEN17["lm_head"]
    say("lm_head argmax 2048->151936, full oracle")
    w = ctx.synth_weight(7, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    idx = ctx.buffer(4 * 4)
    for seed in (1, 2, 3):
        x = oracle.bf16_to_f32(oracle.synth_bf16(seed, 1.0, k)).reshape(1, k)
        ref = oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), 0, n, threads=16)
        xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
        yb = ctx.buffer(n * 4)
        ctx.matmul(xb, mx4.BF16, 1, w, yb)
        ctx.argmax_rows(yb, 1, n, idx)
        y = yb.download(np.float32).reshape(1, n)
        assert_close(y, ref, "lm_head")
        assert int(idx.download(np.uint32, 1)[0]) == oracle.argmax(ref[0])
        assert oracle.argmax(y[0]) == oracle.argmax(ref[0])
        # the fused lm_head + argmax, with and without writing the logits
        y2 = ctx.buffer(n * 4)
        for yy in (y2, None):
            idx.upload(np.full(4, 0xFFFFFFFF, np.uint32))
            ctx.matmul_argmax(xb, mx4.BF16, w, yy, idx)
            assert int(idx.download(np.uint32, 1)[0]) == oracle.argmax(ref[0])
        assert np.array_equal(y2.download(np.float32).reshape(1, n), y)


def test_lm_head_8b_greedy_argmax_identical(mx4, ctx, oracle):
    """The Qwen3-8B lm_head (4096 -> 151936) at M = 1 against the full oracle
    logits, three activation seeds: the logits within the bars, and the greedy
    pick (engine/src/model.rs:228-238 then :288-296) identical through the
    projection + mx4_argmax_rows and through the fused mx4_matmul_argmax, with
    and without writing the logits; the fused launch runs the projection's own
    launch shape (two-wave teams), so the logits it writes are the
    projection's bit for bit."""
    n, k = QWEN8["lm_head"]
    w = ctx.synth_weight(8, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    idx = ctx.buffer(4 * 4)
    for seed in (1, 2, 3):
        say(f"lm_head 8B argmax 4096->151936, full oracle, x seed {seed}")
        x = oracle.bf16_to_f32(oracle.synth_bf16(seed, 1.0, k)).reshape(1, k)
        ref = oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), 0, n, threads=16)
        want = oracle.argmax(ref[0])
        xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
        yb = ctx.buffer(n * 4)
        ctx.matmul(xb, mx4.BF16, 1, w, yb)
        idx.upload(np.full(4, 0xFFFFFFFF, np.uint32))
        ctx.argmax_rows(yb, 1, n, idx)
        y = yb.download(np.float32).reshape(1, n)
        assert_close(y, ref, f"8B lm_head seed {seed}")
        assert int(idx.download(np.uint32, 1)[0]) == want
        assert oracle.argmax(y[0]) == want
        y2 = ctx.buffer(n * 4)
        for yy in (y2, None):
            idx.upload(np.full(4, 0xFFFFFFFF, np.uint32))
            ctx.matmul_argmax(xb, mx4.BF16, w, yy, idx)
            assert int(idx.download(np.uint32, 1)[0]) == want, f"fused, logits {'written' if yy else 'not written'}"
        assert np.array_equal(y2.download(np.float32).reshape(1, n), y), f"8B lm_head fused logits seed {seed}"
    w.release()


def test_lm_head_8b_verify_rows(mx4, ctx, oracle):
    """Speculative verify on the Qwen3-8B lm_head (engine/src/gpu.rs:614-626:
    lm_head over the draft + 1 token rows, then argmax_rows): AUTO at M = 2, 4,
    8, 16 and 32 token rows (few-token GEMV, skinny kernel with the three-tile
    ring, the two-launch split above 16 rows) against the full oracle logits;
    mx4_argmax_rows over the M rows gives the oracle's pick for every row."""
    n, k = QWEN8["lm_head"]
    mmax = 32
    w = ctx.synth_weight(9, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    x = oracle.bf16_to_f32(oracle.synth_bf16(19, 1.0, mmax * k)).reshape(mmax, k)
    say("lm_head 8B verify rows: full oracle logits for 32 token rows")
    ref = oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), 0, n, threads=16)
    want = np.array([oracle.argmax(r) for r in ref], np.uint32)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    yb = ctx.buffer(mmax * n * 4)
    idx = ctx.buffer(mmax * 4)
    for m in (2, 4, 8, 16, 32):
        say(f"lm_head 8B verify m={m}")
        ctx.matmul(xb, mx4.BF16, m, w, yb)
        idx.upload(np.full(mmax, 0xFFFFFFFF, np.uint32))
        ctx.argmax_rows(yb, m, n, idx)
        y = yb.download(np.float32, m * n).reshape(m, n)
        assert_close(y, ref[:m], f"8B lm_head m={m}")
        assert np.array_equal(idx.download(np.uint32, m), want[:m]), m
    w.release()


def test_recorded_decode_tail_replays(mx4, ctx, oracle):
    """A recorded pass (HIP graph) holding the fused lm_head argmax, a separate
    argmax over rows and a few-token GEMV: every replay, with new activations
    uploaded between replays, equals the eager calls on the same inputs (the
    kernels clear nothing with memsets; their key buffers are plain stores)."""
    n, k = 5000, 2048
    w = ctx.synth_weight(61, n, k, 0.02)
    x = ctx.buffer(4 * k * 2)
    y1, idx1, idx2 = ctx.buffer(n * 4), ctx.buffer(4), ctx.buffer(4)
    y4 = ctx.buffer(3 * n * 4)

    def enqueue():
        ctx.matmul_argmax(x, mx4.BF16, w, y1, idx1)
        ctx.argmax_rows(y1, 1, n, idx2)
        ctx.matmul_ptr(x.ptr, mx4.BF16, 3, w, y4.ptr)

    p = ctx.record(enqueue)
    for rep in range(4):
        bits = oracle.synth_bf16(900 + rep, 1.0, 3 * k)
        x.upload(bits)
        p.launch()
        ctx.synchronize()
        got = (y1.download(np.float32), idx1.download(np.uint32)[0], idx2.download(np.uint32)[0],
               y4.download(np.float32))
        enqueue()
        ctx.synchronize()
        want = (y1.download(np.float32), idx1.download(np.uint32)[0], idx2.download(np.uint32)[0],
                y4.download(np.float32))
        assert np.array_equal(got[0], want[0]) and got[1] == want[1] == got[2] == want[2], rep
        assert np.array_equal(got[3], want[3]), rep
        assert got[1] == oracle.argmax(want[0]), rep
    p.release()


@pytest.mark.parametrize("k", [2048, 4096])
def test_matmul_argmax_first_max_rule(mx4, ctx, oracle, k):
    """The fused argmax keeps engine/src/model.rs:288-296 exactly: ties go to the
    lowest row, a maximum in the last row is found, NaN logits never win unless
    in row 0 (then row 0 is the answer), +0 and -0 are equal."""
    n = 3001
    rng = np.random.default_rng(k)
    idx = ctx.buffer(16)

    def run(packed, scales, x, xt=mx4.F32):
        w = ctx.upload_weight(packed, scales, n, k)
        xb = ctx.to_device(np.ascontiguousarray(x, np.float32))
        ctx.matmul_argmax(xb, xt, w, None, idx)
        got = int(idx.download(np.uint32, 1)[0])
        ref = oracle.matmul(np.asarray(x, np.float32).reshape(1, k), packed.reshape(-1), scales.reshape(-1))[0]
        w.release()
        return got, ref

    scales = np.full((n, k // 32), 120, np.uint8)
    x = rng.standard_normal(k).astype(np.float32)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    got, ref = run(packed, scales, x)
    assert got == oracle.argmax(ref)
    # the same maximal row planted at 5, 1700 and the last row: 5 wins; then only the last row
    p2 = packed.copy()
    p2[[5, 1700, n - 1]] = 0x77
    got, ref = run(p2, scales, np.abs(x))
    assert ref[5] == ref[1700] == ref[n - 1] and got == oracle.argmax(ref) == 5
    p3 = packed.copy()
    p3[n - 1] = 0x77
    got, ref = run(p3, scales, np.abs(x))
    assert got == oracle.argmax(ref) == n - 1
    # all-zero weights: every logit is +0 or -0 -> row 0
    got, ref = run(np.zeros_like(packed), scales, x)
    assert got == oracle.argmax(ref) == 0
    # NaN activations: every logit NaN -> row 0
    xn = x.copy()
    xn[3] = np.nan
    got, ref = run(packed, scales, xn)
    assert np.all(np.isnan(ref)) and got == oracle.argmax(ref) == 0


@pytest.mark.parametrize("kind", ["mxfp4", "bf16"])
def test_embed_rows(mx4, ctx, oracle, kind):
    """engine/src/lib.rs:222-227: decoded rows cut to bf16 (low 16 bits dropped),
    bit for bit; ids past the table give zero rows."""
    rows, cols = 777, 2048
    rng = np.random.default_rng(9)
    if kind == "mxfp4":
        w = ctx.synth_weight(55, rows, cols, 0.02)
        packed, scales = ctx.download_weight(w)
        table = (f32_bits(oracle.dequantize(packed, scales)) >> 16).astype(np.uint16)
    else:
        table = rng.integers(0, 1 << 16, (rows, cols), dtype=np.uint16)
        w = ctx.upload_weight_bf16(table, rows, cols)
    ids = np.array([0, rows - 1, 5, 5, 400, rows, 2 ** 31], np.uint32)
    out = ctx.buffer(len(ids) * cols * 2)
    ctx.embed(w, ctx.to_device(ids), len(ids), out)
    got = out.download(np.uint16).reshape(len(ids), cols)
    for t, i in enumerate(ids):
        expected = table[i] if i < rows else np.zeros(cols, np.uint16)
        assert np.array_equal(got[t], expected), (t, i)


def test_argmax_rows_first_max_rule(mx4, ctx, oracle):
    rng = np.random.default_rng(6)
    rows = [rng.standard_normal(151936).astype(np.float32) for _ in range(3)]
    rows[1][[5, 777, 151935]] = 100.0                       # planted ties -> 5
    rows[2][:] = -np.inf                                    # nothing beats column 0
    extra = np.array([np.nan, 9.0, 9.0] + [0.0] * (151936 - 3), np.float32)  # NaN in column 0 -> 0
    x = np.stack(rows + [extra])
    xb, out = ctx.to_device(x), ctx.buffer(4 * 4)
    ctx.argmax_rows(xb, 4, x.shape[1], out)
    got = out.download(np.uint32).tolist()
    assert got == [oracle.argmax(r) for r in x]


@pytest.mark.parametrize("rows,width", [(1, 1), (3, 100), (2, 1024), (2, 1025), (1, 1 << 20), (5, 70001),
                                        (9000, 64), (600, 3000)])
def test_argmax_rows_pieces(mx4, ctx, oracle, rows, width):
    """Rows split over one or many blocks (one launch or keys + reduction),
    with the rule's corner cases planted where pieces meet."""
    rng = np.random.default_rng(rows * 7919 + width)
    x = rng.standard_normal((rows, width)).astype(np.float32)
    x[0, rng.integers(0, width)] = np.nan
    if width > 2:
        r = rows // 2
        x[r, [width // 2, width - 1]] = 50.0                   # tie across pieces -> the lower
        x[r, 0] = np.nan if rows > 1 else x[r, 0]               # NaN in column 0 wins row r
    if rows > 2:
        x[1, :] = -np.inf
        x[1, width - 1] = -0.0
        x[1, width // 3] = 0.0                                  # +0 and -0 tie -> the lower
    if rows > 3:
        x[2, :] = np.nan                                        # all NaN -> 0
        x[3, :] = -np.inf                                       # all -inf -> 0
    xb, out = ctx.to_device(x), ctx.buffer(4 * rows)
    ctx.argmax_rows(xb, rows, width, out)
    got = out.download(np.uint32)
    want = np.array([oracle.argmax(row) for row in x], np.uint32)
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:10]


# ------------------------------------------------------------------ generic / odd shapes

@pytest.mark.parametrize("m,n,k", [(1, 5, 32), (1, 7, 96), (3, 9, 160), (5, 33, 64), (17, 12, 2048),
                                   (33, 40, 256), (1, 300, 8192)])
def test_generic_shapes(mx4, ctx, oracle, m, n, k):
    rng = np.random.default_rng(m * 1000 + n)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(110, 135, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
    for path in (mx4.PATH_AUTO, mx4.PATH_GENERIC):
        y = run_matmul(mx4, ctx, x, w, path)
        assert_close(y, ref, f"m={m} n={n} k={k} path={path}", scaled=True)


def test_errors_are_reported_not_launched(mx4, ctx):
    w = ctx.upload_weight(np.zeros(16, np.uint8), np.array([127], np.uint8), 1, 32)
    x, y = ctx.buffer(64 * 4), ctx.buffer(64 * 4)
    with pytest.raises(mx4.Mx4Error, match="m must be"):
        ctx.matmul(x, mx4.F32, 0, w, y)
    with pytest.raises(mx4.Mx4Error, match="GEMV path"):
        ctx.matmul(x, mx4.F32, 2, w, y, mx4.PATH_GEMV)
    with pytest.raises(mx4.Mx4Error):
        ctx.upload_weight(np.zeros(16, np.uint8), np.array([255], np.uint8), 1, 32)
    with pytest.raises(mx4.Mx4Error, match="divisible"):
        ctx.upload_weight(np.zeros(16, np.uint8), np.array([127], np.uint8), 1, 31)


def test_weights_outlive_their_context(mx4, oracle):
    """mx4_destroy detaches the caller's weight handles (the Rust Tensor owns
    its GpuTensor, engine/src/gpu.rs:225-237, and may drop it after the
    backend): their device memory is freed with the context, every entry point
    then refuses them, and mx4_weight_release afterwards frees only the handle.
    Covers an uploaded weight with its matrix-core copy, a bf16 weight and a
    wrapped one; a fresh context on the same device works as before."""
    import ctypes

    L = mx4.lib()
    n, k = 64, 256
    rng = np.random.default_rng(31)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(120, 130, (n, k // 32), dtype=np.uint8)
    h = ctypes.c_void_p()
    mx4.check(L.mx4_create(0, ctypes.byref(h)))
    dead = h.value
    ws = []
    w = ctypes.c_void_p()
    mx4.check(L.mx4_weight_upload(dead, packed.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                                  scales.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), n, k, ctypes.byref(w)))
    ws.append(w.value)
    mx4.check(L.mx4_weight_prepare_prefill(w.value))
    bits = rng.integers(0, 1 << 15, (n, k), dtype=np.uint16)
    wb = ctypes.c_void_p()
    mx4.check(L.mx4_weight_upload_bf16(dead, bits.ctypes.data, n, k, ctypes.byref(wb)))
    ws.append(wb.value)
    mem = ctypes.c_void_p()
    mx4.check(L.mx4_malloc(dead, n * k // 2 + 256 + n * k // 32, ctypes.byref(mem)))
    mx4.check(L.mx4_upload(dead, mem, packed.ctypes.data, n * k // 2))
    mx4.check(L.mx4_upload(dead, ctypes.c_void_p(mem.value + n * k // 2 + 256), scales.ctypes.data, n * k // 32))
    ww = ctypes.c_void_p()
    mx4.check(L.mx4_weight_wrap(dead, mem, ctypes.c_void_p(mem.value + n * k // 2 + 256), n, k, ctypes.byref(ww)))
    ws.append(ww.value)
    mx4.check(L.mx4_synchronize(dead))
    mx4.check(L.mx4_free(dead, mem))  # the wrapped weight's memory is the caller's
    L.mx4_destroy(dead)
    with mx4.Context(0) as fresh:
        x = fresh.to_device(np.ones(k, np.float32))
        y = fresh.buffer(n * 4)
        for i, wh in enumerate(ws):
            rows = ctypes.c_uint32()
            st = L.mx4_weight_info(wh, ctypes.byref(rows), None, None, None)
            assert st == 1 and "destroyed" in L.mx4_last_error().decode(), f"weight {i}: info after destroy"
            st = L.mx4_matmul(fresh.handle, x.ptr, mx4.F32, 1, wh, y.ptr)
            assert st == 1 and "destroyed" in L.mx4_last_error().decode(), f"weight {i}: matmul after destroy"
            assert L.mx4_weight_prepare_prefill(wh) == 1
        for wh in ws:
            L.mx4_weight_release(wh)  # frees the handle only
        # the device is unaffected: a new weight on the fresh context multiplies correctly
        w2 = fresh.upload_weight(packed, scales, n, k)
        xv = oracle.bf16_to_f32(oracle.synth_bf16(32, 1.0, k)).reshape(1, k)
        got = run_matmul(mx4, fresh, xv, w2, mx4.PATH_AUTO)
        assert_close(got, oracle.matmul(xv, packed.reshape(-1), scales.reshape(-1)), "weight after destroy cycle")
        w2.release()


# ------------------------------------------------------------------ kernel configurations

CONFIG_SHAPES = [(1000, 2048), (1000, 4096), (700, 6144), (999, 8192), (700, 12288)]


@pytest.mark.parametrize("n,k", CONFIG_SHAPES)
def test_gemv_every_configuration(mx4, ctx, oracle, n, k):
    """Every instantiated (team, rows, teams, teams per workgroup) of the M = 1 kernel
    agrees with the oracle, including ragged tails (n not a multiple of the rows per
    team) and workgroups whose later teams run past the last row-set."""
    say(f"gemv configurations {k}->{n}")
    w = ctx.synth_weight(77, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    xb16 = oracle.synth_bf16(3, 1.0, k)
    x = oracle.bf16_to_f32(xb16).reshape(1, k)
    ref = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
    xdev = {mx4.BF16: ctx.to_device(xb16), mx4.F32: ctx.to_device(x)}
    y = ctx.buffer(n * 4)
    nblk = k // 32
    tried = 0
    for team in (1, 2, 3, 4, 6):
        if nblk % (64 * team):
            continue
        bpl = nblk // (64 * team)
        for rows in (1, 2, 4, 8):
            if rows * bpl > 8:
                continue
            for teams in (0, 1, 7, 64):
                for tpw in (1, 2, 4, 8):
                    if 64 * team * tpw > 512:
                        continue
                    for xt in (mx4.BF16, mx4.F32):
                        if tpw > 1 and k * (2 if xt == mx4.BF16 else 4) + tpw * 2 * team * rows * 4 > 65536:
                            continue
                        y.upload(np.full(n, np.nan, np.float32))
                        ctx.gemv_config(xdev[xt].ptr, xt, w, y.ptr, team, rows, teams, tpw)
                        got = y.download(np.float32).reshape(1, n)
                        assert_close(got, ref, f"team={team} rows={rows} teams={teams} tpw={tpw} xt={xt}")
                        tried += 1
    assert tried >= 64


def test_gemv_writes_every_row_each_launch(mx4, ctx, oracle):
    """Every M = 1 GEMV launch writes every row of y, whatever its launch shape:
    the 8B q|k|v and gate|up groups and o, the 1.7B o and k, and explicit
    configurations (fewer teams than rows, several rows per team, several
    teams per workgroup, the last workgroup partly empty) run interleaved, 12
    rounds eagerly and then 4 replays of one recorded pass, each into a y first
    overwritten with NaN. Every launch must leave no NaN, equal the first
    launch bit for bit, and that result is the oracle's."""
    import ctypes

    L = mx4.lib()
    rng = np.random.default_rng(47)
    specs = [("8B q|k|v", [(4096, 4096), (1024, 4096), (1024, 4096)], None),
             ("8B o", [(4096, 4096)], None),
             ("8B gate|up", [(12288, 4096), (12288, 4096)], None),
             ("1.7B o", [(2048, 2048)], None),
             ("1.7B k", [(1024, 2048)], None),
             ("33 teams of 1 row", [(1000, 4096)], (1, 1, 33, 1)),
             ("100 teams of 4 rows, 2 per workgroup", [(3001, 2048)], (1, 4, 100, 2)),
             ("8 teams per workgroup, 2 rows", [(5000, 2048)], (1, 2, 600, 8))]
    cases = []
    seed = 700
    for name, dims, cfg in specs:
        k = dims[0][1]
        ws = []
        for n, _ in dims:
            ws.append(ctx.synth_weight(seed, n, k, 0.02))
            seed += 1
        xv = oracle.bf16_to_f32(oracle.synth_bf16(seed, 1.0, k)).reshape(1, k)
        xb = ctx.to_device((f32_bits(xv) >> 16).astype(np.uint16))
        ys = [ctx.buffer(n * 4) for n, _ in dims]
        nans = [ctx.to_device(np.full(n, np.nan, np.float32)) for n, _ in dims]
        refs = []
        for w, (n, _) in zip(ws, dims):
            packed, scales = ctx.download_weight(w)
            refs.append(oracle.matmul_rows(xv, packed.reshape(-1), scales.reshape(-1), 0, n, threads=8))
        cases.append((name, ws, xb, ys, nans, refs, cfg))

    def enqueue(case):
        name, ws, xb, ys, nans, refs, cfg = case
        for y, nan in zip(ys, nans):
            mx4.check(L.mx4_copy(ctx.handle, ctypes.c_void_p(y.ptr), ctypes.c_void_p(nan.ptr), y.nbytes))
        if cfg is not None:
            ctx.gemv_config(xb.ptr, mx4.BF16, ws, [y.ptr for y in ys], team=cfg[0], rows=cfg[1], teams=cfg[2],
                            tpw=cfg[3])
        elif len(ws) == 1:
            ctx.matmul_ptr(xb.ptr, mx4.BF16, 1, ws[0], ys[0].ptr)
        else:
            ctx.matmul_group(xb.ptr, mx4.BF16, 1, ws, [y.ptr for y in ys])

    first = {}
    for rnd in range(12):
        order = list(range(len(cases)))
        rng.shuffle(order)
        for ci in order:
            enqueue(cases[ci])
            ctx.synchronize()
            name, _, _, ys, _, refs, _ = cases[ci]
            got = [y.download(np.float32) for y in ys]
            for i, g in enumerate(got):
                assert not np.any(np.isnan(g)), f"{name} round {rnd}: segment {i} has rows no team wrote"
            if name not in first:
                first[name] = got
                for i, (g, r) in enumerate(zip(got, refs)):
                    assert_close(g.reshape(1, -1), r, f"{name} segment {i}")
            else:
                for i, (g, f) in enumerate(zip(got, first[name])):
                    assert np.array_equal(f32_bits(g), f32_bits(f)), f"{name} round {rnd}: segment {i} differs"
    p = ctx.record(lambda: [enqueue(c) for c in cases])
    for rep in range(4):
        p.launch()
        ctx.synchronize()
        for name, _, _, ys, _, _, _ in cases:
            for i, y in enumerate(ys):
                assert np.array_equal(f32_bits(y.download(np.float32)), f32_bits(first[name][i])), \
                    f"{name} replay {rep}: segment {i}"
    p.release()
    for c in cases:
        for w in c[1]:
            w.release()


def test_group_equals_individual(mx4, ctx, oracle):
    """q|k|v and gate|up as one launch give bitwise the same rows as separate launches."""
    k = 4096
    shapes = [4096, 1024, 1024]
    ws = [ctx.synth_weight(200 + i, n, k, 0.02) for i, n in enumerate(shapes)]
    xb = ctx.to_device(oracle.synth_bf16(5, 1.0, k))
    ys = [ctx.buffer(n * 4) for n in shapes]
    ctx.matmul_group(xb.ptr, mx4.BF16, 1, ws, [y.ptr for y in ys])
    grouped = [y.download(np.float32) for y in ys]
    for w, y, g in zip(ws, ys, grouped):
        ctx.matmul_ptr(xb.ptr, mx4.BF16, 1, w, y.ptr)
        assert np.array_equal(f32_bits(y.download(np.float32)), f32_bits(g))
    with pytest.raises(mx4.Mx4Error, match="share their width"):
        other = ctx.synth_weight(9, 64, 2048, 0.02)
        ctx.matmul_group(xb.ptr, mx4.BF16, 1, [ws[0], other], [ys[0].ptr, ys[1].ptr])


@pytest.mark.parametrize("k,shapes", [
    (4096, [4096, 1024, 1024]),    # 8B q|k|v: every team starts in q (preloaded head), later turns reach k and v
    (4096, [12288, 12288]),        # 8B gate|up: preloaded head, 8 teams per workgroup
    (4096, [3001, 999, 7]),        # preloaded head, ragged row-sets at every segment end
    (2048, [2048, 1024, 1024]),    # 1.7B q|k|v: more teams than q's row-sets, the table kernel
    (2048, [6144, 6144]),          # 1.7B gate|up: the table kernel
    (4096, [40, 8, 24, 100]),      # four tiny segments: one row-set per team, the table kernel
    (12288, [2050, 30]),           # wide K, 3-wave teams
])
def test_group_segments_against_oracle(mx4, ctx, oracle, k, shapes):
    """A grouped launch equals the separate launches bit for bit and the oracle to
    the float bar, for bf16 and f32 activations. The launcher passes segment 0's
    fields as preloaded scalars when every team's first row-set lies in segment 0
    (teams <= segment 0's row-sets) and the whole table otherwise; the cases above
    take both kernels."""
    say(f"grouped gemv k={k} shapes={shapes}")
    ws = [ctx.synth_weight(300 + i, n, k, 0.02) for i, n in enumerate(shapes)]
    xb16 = oracle.synth_bf16(11, 1.0, k)
    x = oracle.bf16_to_f32(xb16).reshape(1, k)
    xdev = {mx4.BF16: ctx.to_device(xb16), mx4.F32: ctx.to_device(x)}
    refs = []
    for w in ws:
        packed, scales = ctx.download_weight(w)
        refs.append(oracle.matmul(x, packed.reshape(-1), scales.reshape(-1)))
    ys = [ctx.buffer(n * 4) for n in shapes]
    for xt in (mx4.BF16, mx4.F32):
        for y, n in zip(ys, shapes):
            y.upload(np.full(n, np.nan, np.float32))
        ctx.matmul_group(xdev[xt].ptr, xt, 1, ws, [y.ptr for y in ys])
        grouped = [y.download(np.float32) for y in ys]
        for i, (w, y, g, ref) in enumerate(zip(ws, ys, grouped, refs)):
            assert_close(g.reshape(1, -1), ref, f"segment {i} xt={xt}")
            ctx.matmul_ptr(xdev[xt].ptr, xt, 1, w, y.ptr)
            assert np.array_equal(f32_bits(y.download(np.float32)), f32_bits(g)), f"segment {i} xt={xt}"


GROUP_FEW = [
    (4096, [4096, 1024, 1024], (2, 3, 8, 17, 32)),  # 8B q|k|v: few-token GEMV at 2, skinny above, two launches past 16
    (4096, [12288, 12288], (2, 4, 8, 20, 32)),      # 8B gate|up: the tile ring; from 20 tokens one split-K launch
    (4096, [501, 299, 7], (3, 4)),                  # 807 rows: the few-token GEMV at 3-4 tokens, ragged row-sets
    (4096, [1000, 70, 70], (3, 5, 16)),             # 1140 rows: skinny, a ragged tile at every weight's end
    (2048, [2048, 1024, 1024], (2, 4, 8, 24)),      # 1.7B q|k|v
    (4096, [40, 8, 24, 100], (2, 5, 16)),           # four tiny weights, 13 tiles
]


@pytest.mark.parametrize("k,shapes,ms", GROUP_FEW, ids=[f"k{k}-{'_'.join(map(str, s))}" for k, s, _ in GROUP_FEW])
def test_group_few_tokens_against_oracle(mx4, ctx, oracle, k, shapes, ms):
    """2..32 token rows through mx4_matmul_group: a verify step's q|k|v or
    gate|up as one launch of the few-token GEMV or the skinny kernel, each
    weight a run of row-sets or 16-row tiles of it. Every weight's outputs
    against the oracle (on weights wider than 1024 rows: their first and last
    16 rows and 64 drawn), and against separate mx4_matmul calls within f32
    rounding; outputs start as NaN, so a tile written to the wrong weight, or
    not written, shows. bf16 activations, and f32 ones (the skinny kernel's
    three-term split) on the small groups."""
    rng = np.random.default_rng(k + len(shapes))
    ws = [ctx.synth_weight(400 + i, n, k, 0.02) for i, n in enumerate(shapes)]
    dl = [ctx.download_weight(w) for w in ws]
    rows = [np.arange(n) if n <= 1024 else np.unique(np.r_[0:16, n - 16:n, rng.choice(n, 64)]) for n in shapes]
    for m in ms:
        xb16 = oracle.synth_bf16(410 + m, 1.0, m * k)
        x = oracle.bf16_to_f32(xb16).reshape(m, k)
        xts = [mx4.BF16] + ([mx4.F32] if sum(shapes) <= 2048 and m >= 3 else [])
        for xt in xts:
            say(f"grouped few tokens k={k} shapes={shapes} m={m} xt={xt}")
            xd = ctx.to_device(xb16 if xt == mx4.BF16 else x)
            ys = [ctx.buffer(m * n * 4) for n in shapes]
            for y, n in zip(ys, shapes):
                y.upload(np.full(m * n, np.nan, np.float32))
            ctx.matmul_group(xd.ptr, xt, m, ws, [y.ptr for y in ys])
            grouped = [y.download(np.float32).reshape(m, n) for y, n in zip(ys, shapes)]
            for i, ((packed, scales), n, g, r) in enumerate(zip(dl, shapes, grouped, rows)):
                assert np.all(np.isfinite(g)), f"weight {i} m={m}: rows left unwritten"
                ref = oracle.matmul(x, packed[r].reshape(-1), scales[r].reshape(-1))
                assert_close(g[:, r], ref, f"grouped weight {i} m={m} xt={xt}")
                ctx.matmul_ptr(xd.ptr, xt, m, ws[i], ys[i].ptr)
                assert_close(g, ys[i].download(np.float32).reshape(m, n), f"grouped vs separate {i} m={m} xt={xt}")
            for y in ys:
                y.free()
            xd.free()
    for w in ws:
        w.release()


GROUP_EXACT = [
    (4096, [4096, 1024, 1024], (40, 128, 512)),  # 8B q|k|v (at 40 rows fewer tiles than CUs)
    (4096, [12288, 12288], (64,)),               # 8B gate|up
    (4096, [1000, 300, 77], (200,)),             # ragged column tiles at every weight's end
]


@pytest.mark.parametrize("k,shapes,ms", GROUP_EXACT, ids=[f"k{k}-{'_'.join(map(str, s))}" for k, s, _ in GROUP_EXACT])
def test_group_exact_gemm_against_oracle(mx4, ctx, oracle, k, shapes, ms):
    """More than 32 token rows through mx4_matmul_group: one exact-GEMM launch
    over every weight's column tiles, K unsplit. Each weight's outputs against the
    oracle (first and last 16 rows and 48 drawn on weights wider than 1024)
    and against separate mx4_matmul calls, bf16 and f32 activations, outputs
    NaN-filled first."""
    rng = np.random.default_rng(k + sum(shapes))
    ws = [ctx.synth_weight(440 + i, n, k, 0.02) for i, n in enumerate(shapes)]
    dl = [ctx.download_weight(w) for w in ws]
    rows = [np.arange(n) if n <= 1024 else np.unique(np.r_[0:16, n - 16:n, rng.choice(n, 48)]) for n in shapes]
    for m in ms:
        xb16 = oracle.synth_bf16(450 + m, 1.0, m * k)
        x = oracle.bf16_to_f32(xb16).reshape(m, k)
        for xt in (mx4.BF16, mx4.F32):
            say(f"grouped exact GEMM k={k} shapes={shapes} m={m} xt={xt}")
            xd = ctx.to_device(xb16 if xt == mx4.BF16 else x)
            ys = [ctx.buffer(m * n * 4) for n in shapes]
            for y, n in zip(ys, shapes):
                y.upload(np.full(m * n, np.nan, np.float32))
            ctx.matmul_group(xd.ptr, xt, m, ws, [y.ptr for y in ys])
            grouped = [y.download(np.float32).reshape(m, n) for y, n in zip(ys, shapes)]
            for i, ((packed, scales), n, g, r) in enumerate(zip(dl, shapes, grouped, rows)):
                assert np.all(np.isfinite(g)), f"weight {i} m={m}: outputs left unwritten"
                ref = oracle.matmul(x, packed[r].reshape(-1), scales[r].reshape(-1))
                assert_close(g[:, r], ref, f"grouped exact weight {i} m={m} xt={xt}")
                ctx.matmul_ptr(xd.ptr, xt, m, ws[i], ys[i].ptr)
                assert_close(g, ys[i].download(np.float32).reshape(m, n), f"grouped vs separate {i} m={m} xt={xt}")
            for y in ys:
                y.free()
            xd.free()
    for w in ws:
        w.release()


def test_group_few_tokens_replayed(mx4, ctx, oracle):
    """Grouped verify launches recorded in a pass and replayed three times, the
    program's own synchronizations between replays: every replay gives the
    eager call's bits, for the few-token GEMV (2 tokens), the tile ring (8)
    and the split-K launch whose arrival counts each launch re-arms (24
    tokens on ring-length weights)."""
    k = 4096
    shapes = [12288, 12288]
    ws = [ctx.synth_weight(420 + i, n, k, 0.02) for i, n in enumerate(shapes)]
    for m in (2, 8, 24):
        say(f"grouped few tokens replayed m={m}")
        xd = ctx.to_device(oracle.synth_bf16(430 + m, 1.0, m * k))
        ys = [ctx.buffer(m * n * 4) for n in shapes]

        def run():
            ctx.matmul_group(xd.ptr, mx4.BF16, m, ws, [y.ptr for y in ys])

        run()
        eager = [y.download(np.float32).view(np.uint32) for y in ys]
        p = ctx.record(run)
        for _ in range(3):
            for y, n in zip(ys, shapes):
                y.upload(np.full(m * n, np.nan, np.float32))
            p.launch()
            ctx.synchronize()
            for y, e in zip(ys, eager):
                assert np.array_equal(y.download(np.float32).view(np.uint32), e), m
        p.release()
        for y in ys:
            y.free()
        xd.free()
    for w in ws:
        w.release()


def test_extreme_scales_take_the_exact_path(mx4, ctx, oracle):
    """Scale bytes 0, 1 (subnormal weights) and 253, 254 (inf weights) are outside
    the converter-folding range; AUTO routes them to the exact generic kernel."""
    rng = np.random.default_rng(8)
    n, k = 64, 4096
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(118, 130, (n, k // 32), dtype=np.uint8)
    scales[0:8, 3] = 0
    scales[8:16, 5] = 1
    x = oracle.bf16_to_f32(oracle.synth_bf16(4, 1.0, k)).reshape(1, k)
    w = ctx.upload_weight(packed, scales, n, k)
    ref = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
    y = run_matmul(mx4, ctx, x, w, mx4.PATH_AUTO, mx4.BF16)
    assert_close(y, ref, "subnormal scales", scaled=True)
    with pytest.raises(mx4.Mx4Error, match="2..252"):
        run_matmul(mx4, ctx, x, w, mx4.PATH_GEMV, mx4.BF16)
    # a row made only of scale-0 blocks: every weight is subnormal, exact products
    scales2 = scales.copy()
    scales2[20, :] = 0
    w2 = ctx.upload_weight(packed, scales2, n, k)
    y2 = run_matmul(mx4, ctx, x, w2, mx4.PATH_AUTO, mx4.F32)
    ref2 = oracle.matmul(x, packed.reshape(-1), scales2.reshape(-1))
    assert abs(float(y2[0, 20]) - float(ref2[0, 20])) <= 1e-3 * abs(float(ref2[0, 20])) + 1e-44
    # overflowing weights: inf and NaN patterns match the oracle's
    scales3 = scales.copy()
    scales3[30, 0] = 254
    scales3[31, 0] = 253
    w3 = ctx.upload_weight(packed, scales3, n, k)
    y3 = run_matmul(mx4, ctx, x, w3, mx4.PATH_AUTO, mx4.F32)
    ref3 = oracle.matmul(x, packed.reshape(-1), scales3.reshape(-1))
    assert np.array_equal(np.isnan(y3), np.isnan(ref3)) and np.array_equal(np.isinf(y3), np.isinf(ref3))
    fin = np.isfinite(ref3)
    assert_close(y3[fin].reshape(1, -1), ref3[fin].reshape(1, -1), "finite rows next to inf rows", scaled=True)


@pytest.mark.parametrize("path,m", [("GEMV", 1), ("SKINNY", 8), ("GEMM", 40), ("AUTO", 40)])
def test_f32_activations_inf_nan_and_huge(mx4, ctx, oracle, path, m):
    """f32 token rows holding +inf, -inf, NaN or a huge finite value
    (3.4e38, above the point where rounding to bf16 would give inf), through
    the exact f32-activation paths (the GEMV's f32 FMA, and the bf16 matrix
    cores with x split into three bf16 terms in the skinny kernel and the
    GEMM). The reference's f32 loop (engine/src/lib.rs:240-266) gives +-inf
    where the weight is nonzero and NaN where it is zero (inf * 0), NaN for a
    NaN row, and finite sums for the huge row: the NaN/inf pattern must be the
    oracle's exactly, and every finite row within the usual bars."""
    rng = np.random.default_rng(17 + m)
    n, k = 256, 4096
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(118, 125, (n, k // 32), dtype=np.uint8)  # |w| <= 0.75: huge * w stays finite
    w = ctx.upload_weight(packed, scales, n, k)
    cases = [("+inf", 5, np.inf), ("-inf", 9, -np.inf), ("nan", 11, np.nan), ("huge", 7, np.float32(3.4e38))]
    # several token rows: one special row each, in a single call; one row: a call per case
    plans = [dict(enumerate(cases))] if m >= len(cases) else [{0: c} for c in cases]
    for pi, special in enumerate(plans):
        x = oracle.bf16_to_f32(oracle.synth_bf16(18 + pi, 1.0, m * k)).reshape(m, k).copy()
        for row, (_, col, v) in special.items():
            x[row, col] = v
        ref = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
        say(f"f32 non-finite activations path {path} m {m} plan {pi}")
        y = run_matmul(mx4, ctx, x, w, getattr(mx4, f"PATH_{path}"), mx4.F32)
        for row, (label, _, _) in special.items():
            if label == "huge":
                assert np.all(np.isfinite(ref[row])), "the huge row's reference must be finite"
                assert_close(y[row:row + 1], ref[row:row + 1], f"{path} huge finite row", scaled=True)
            else:
                assert np.array_equal(np.isnan(y[row]), np.isnan(ref[row])), f"{path} {label} row: NaN pattern"
                assert np.array_equal(np.isposinf(y[row]), np.isposinf(ref[row])), f"{path} {label}: +inf pattern"
                assert np.array_equal(np.isneginf(y[row]), np.isneginf(ref[row])), f"{path} {label}: -inf pattern"
        plain = [r for r in range(m) if r not in special]
        if plain:
            assert_close(y[plain], ref[plain], f"{path} finite rows next to non-finite ones")


# ------------------------------------------------------------------ skinny (speculative verify)

@pytest.mark.parametrize("name", ["k", "q", "gate", "down"])
def test_skinny_8b_shapes(mx4, ctx, oracle, name):
    """M = 1..32 token rows (draft length + 1 and beyond) on the exact skinny kernel,
    bf16 and f32 activations, sampled weight rows against the oracle."""
    n, k = QWEN8[name]
    say(f"skinny 8B {name} {k}->{n}")
    rng = np.random.default_rng(11)
    w = ctx.synth_weight(300, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    rows = _sample_rows(n, 160, rng)
    for m in (1, 2, 3, 4, 5, 8, 9, 12, 16, 17, 24, 32):
        xbits = oracle.synth_bf16(40 + m, 1.0, m * k)
        x = oracle.bf16_to_f32(xbits).reshape(m, k)
        ref = np.concatenate([oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), int(r), int(r) + 1)
                              for r in rows], axis=1)
        for xtype in (mx4.BF16, mx4.F32):
            xin = x if xtype == mx4.BF16 else (x + rng.standard_normal(x.shape).astype(np.float32) * 1e-3)
            refx = ref if xtype == mx4.BF16 else np.concatenate(
                [oracle.matmul_rows(xin, packed.reshape(-1), scales.reshape(-1), int(r), int(r) + 1) for r in rows], axis=1)
            path = mx4.PATH_SKINNY if m == 1 else mx4.PATH_AUTO
            y = run_matmul(mx4, ctx, xin, w, path, xtype)
            assert_close(y[:, rows], refx, f"skinny {name} m={m} xtype={xtype}")


@pytest.mark.parametrize("n,k", [(2048, 2048), (2048, 6144), (1000, 6144), (333, 2048)])
def test_skinny_resident_activations(mx4, ctx, oracle, n, k):
    """The skinny kernel with bf16 activations held in registers for the whole
    kernel (K up to 6144: the 1.7B q/o/gate/up and down widths; an odd number of
    units per tile at 6144), including ragged N, against the oracle; f32
    activations (the per-tile loading form) on the same weights."""
    say(f"skinny resident x {k}->{n}")
    rng = np.random.default_rng(n + k)
    w = ctx.synth_weight(1100 + k // 1024, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    rows = _sample_rows(n, 96, rng) if n > 96 else np.arange(n)
    for m in (5, 8, 16, 17):
        x = oracle.bf16_to_f32(oracle.synth_bf16(1200 + m, 1.0, m * k)).reshape(m, k)
        ref = np.concatenate([oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), int(r), int(r) + 1)
                              for r in rows], axis=1)
        for xtype in (mx4.BF16, mx4.F32):
            y = run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, xtype)
            assert_close(y[:, rows], ref, f"skinny {k}->{n} m={m} xtype={xtype}")


@pytest.mark.parametrize("n", [333, 4096 + 5, 8192 + 37])
def test_skinny_lds_activations(mx4, ctx, oracle, n):
    """K = 12288 with 1..16 bf16 token rows: the skinny kernel keeps the
    activations in LDS (padded rows; all of K up to 5 tokens, K halves up to
    10, thirds up to 16, each slice loaded when its first unit comes up) and
    reads
    each unit's operand fragments from there. Ragged N against the oracle on
    every row (several 16-row tiles per workgroup on the wider N, so every
    slice is reloaded per tile), and one-hot activations (one column per token,
    drawn across all slices) return the decoded weights bit for bit, which pins
    the LDS row, slice and element placement; f32 activations (the per-unit
    loading form) on the same weights."""
    k = 12288
    say(f"skinny LDS x {k}->{n}")
    rng = np.random.default_rng(n)
    w = ctx.synth_weight(1300 + n % 7, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    for m in (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16):
        x = oracle.bf16_to_f32(oracle.synth_bf16(1310 + m, 1.0, m * k)).reshape(m, k)
        ref = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
        assert_close(run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, mx4.BF16), ref, f"skinny LDS x m={m} n={n}")
        if m in (5, 16):
            assert_close(run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, mx4.F32), ref, f"skinny f32 x m={m} n={n}")
    p2 = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s2 = rng.integers(110, 140, (n, k // 32), dtype=np.uint8)
    w2 = ctx.upload_weight(p2, s2, n, k)
    dec = oracle.dequantize(p2, s2)
    for m in (1, 3, 5, 7, 10, 11, 13, 16):
        cols = rng.choice(k, m, replace=False)
        x = np.zeros((m, k), np.float32)
        x[np.arange(m), cols] = 1.0
        y = run_matmul(mx4, ctx, x, w2, mx4.PATH_SKINNY, mx4.BF16)
        assert np.array_equal(y, dec[:, cols].T), m


@pytest.mark.parametrize("k", [2048, 4096, 6144, 8192, 12288])
def test_gemv_few_tokens(mx4, ctx, oracle, k):
    """2 <= M <= 4 bf16 token rows on the decode GEMV path (the weights read once
    for all of them): ragged N against the oracle, and one-hot activations
    return the decoded weights bit for bit."""
    say(f"few-token GEMV k={k}")
    rng = np.random.default_rng(k)
    n = 333
    w = ctx.synth_weight(700 + k // 1024, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    for m in (2, 3, 4):
        x = oracle.bf16_to_f32(oracle.synth_bf16(800 + m, 1.0, m * k)).reshape(m, k)
        ref = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
        assert_close(run_matmul(mx4, ctx, x, w, mx4.PATH_GEMV, mx4.BF16), ref, f"few-token m={m} k={k}")
    p2 = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s2 = rng.integers(110, 140, (n, k // 32), dtype=np.uint8)
    w2 = ctx.upload_weight(p2, s2, n, k)
    for m in (2, 3, 4):
        cols = rng.choice(k, m, replace=False)
        x = np.zeros((m, k), np.float32)
        x[np.arange(m), cols] = 1.0
        y = run_matmul(mx4, ctx, x, w2, mx4.PATH_GEMV, mx4.BF16)
        assert np.array_equal(y, oracle.dequantize(p2, s2)[:, cols].T), m


@pytest.mark.parametrize("n,k", [(8192 + 5, 4096), (16384 + 37, 2048)])
def test_skinny_tile_ring(mx4, ctx, oracle, n, k):
    """Weights long enough for the skinny kernel's three-tile ring (at least two
    16-row tiles per workgroup at eight waves per CU), ragged N, up to 16 tokens
    in one launch and more as two: one-hot bf16 activations return the decoded
    weights bit for bit in every row, and random activations match the oracle on
    sampled rows."""
    say(f"skinny tile ring {k}->{n}")
    rng = np.random.default_rng(n)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(112, 136, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    dec = oracle.dequantize(packed, scales)
    for m in (5, 16, 17, 32):
        cols = rng.choice(k, m, replace=False)
        x = np.zeros((m, k), np.float32)
        x[np.arange(m), cols] = 1.0
        y = run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, mx4.BF16)
        assert np.array_equal(y, dec[:, cols].T), f"identity m={m}"
    rows = _sample_rows(n, 128, rng)
    for m in (8, 13, 29):
        x = oracle.bf16_to_f32(oracle.synth_bf16(1500 + m, 1.0, m * k)).reshape(m, k)
        ref = np.concatenate([oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), int(r), int(r) + 1)
                              for r in rows], axis=1)
        y = run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, mx4.BF16)
        assert_close(y[:, rows], ref, f"ring {k}->{n} m={m}", scaled=True)


@pytest.mark.parametrize("n,k", [(4096 + 5, 12288), (8192 + 37, 12288), (1024 - 5, 4096), (4096 + 5, 4096),
                                 (8192 + 5, 4096)])
def test_skinny_split_k(mx4, ctx, oracle, n, k):
    """Split K with bf16 activations: K = 12288 from 17 tokens on (four
    workgroups per 16-row tile, each over a quarter of K; up to 16 tokens the
    activations sit in LDS instead), K = 4096 from 17 on
    (four slices when every CU gets one tile, as for 1019 rows; two from 20
    tokens on for weights long enough for the tile ring, as 8197 rows; 4101
    rows stay unsplit); the last workgroup of a tile adds the partials (fewer
    tokens run unsplit, on the same weights). One-hot
    activations return every decoded weight row bit for bit (a tile whose sum
    went missing would show), random activations match the oracle on sampled
    rows, a repeated call is bit-identical (the arrival counts are re-armed),
    and 17-32 tokens on 8229 x 12288 (more partial tiles than the context's
    scratch holds) run unsplit with the same results."""
    say(f"skinny split K {k}->{n}")
    rng = np.random.default_rng(n)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(112, 136, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    dec = oracle.dequantize(packed, scales)
    for m in (1, 8, 16, 17, 32):
        cols = rng.choice(k, m, replace=False)
        x = np.zeros((m, k), np.float32)
        x[np.arange(m), cols] = 1.0
        y = run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, mx4.BF16)
        assert np.array_equal(y, dec[:, cols].T), f"identity m={m}"
    rows = _sample_rows(n, 128, rng)
    for m in (5, 12, 29):
        x = oracle.bf16_to_f32(oracle.synth_bf16(1700 + m, 1.0, m * k)).reshape(m, k)
        ref = np.concatenate([oracle.matmul_rows(x, packed.reshape(-1), scales.reshape(-1), int(r), int(r) + 1)
                              for r in rows], axis=1)
        y = run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, mx4.BF16)
        assert_close(y[:, rows], ref, f"split K {k}->{n} m={m}", scaled=True)
        assert np.array_equal(run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, mx4.BF16), y), f"repeat m={m}"


def test_skinny_ragged_rows_and_identity(mx4, ctx, oracle):
    """Weight rows not a multiple of the 16-row tile, and an exact identity KAT:
    one-hot activations return the decoded weights bit for bit."""
    rng = np.random.default_rng(12)
    n, k = 37, 2048
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(110, 140, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    m = 16
    x = np.zeros((m, k), np.float32)
    cols = rng.choice(k, m, replace=False)
    x[np.arange(m), cols] = 1.0
    for xtype in (mx4.BF16, mx4.F32):
        y = run_matmul(mx4, ctx, x, w, mx4.PATH_SKINNY, xtype)
        dec = oracle.dequantize(packed, scales)
        assert np.array_equal(y, dec[:, cols].T), xtype
    x2 = rng.standard_normal((5, k)).astype(np.float32)
    ref = oracle.matmul(x2, packed.reshape(-1), scales.reshape(-1))
    assert_close(run_matmul(mx4, ctx, x2, w, mx4.PATH_AUTO, mx4.F32), ref, "ragged f32", scaled=True)


# ------------------------------------------------------------------ prefill (block-scaled MFMA)

# ------------------------------------------------------------------ exact GEMM (M > 32)

GEMM_INSTANCES = [(2, 2, 2, 3), (2, 2, 2, 2), (2, 2, 2, 1), (2, 2, 1, 2), (4, 1, 1, 2), (2, 2, 1, 1), (1, 4, 2, 2),
                  (1, 4, 2, 1), (1, 4, 1, 2), (1, 4, 1, 1), (2, 4, 2, 2), (2, 4, 1, 2)]
GEMM_BF16_ONLY = {(2, 4, 2, 2)}  # its f32 tile would leave LDS room for one stage only


@pytest.mark.parametrize("ks", [1, 2, 4])
@pytest.mark.parametrize("inst", GEMM_INSTANCES, ids=[f"{a}x{b}w-{c}x{d}t" for a, b, c, d in GEMM_INSTANCES])
def test_gemm_identity_and_oracle_every_instance(mx4, ctx, oracle, inst, ks):
    """The exact tiled GEMM (bf16 MFMA, weights decoded on the way from LDS),
    every compiled instance on ragged M and N, unsplit and with K split across
    2 and 4 workgroups (partials added in slice order by a second kernel):
    one-hot activations return the decoded weights bit for bit (pins the
    operand and output layouts, the folded scales and the slice offsets),
    random bf16 and f32 activations match the oracle, and a repeated call is
    bit-identical."""
    wm, wn, tm, tn = inst
    rng = np.random.default_rng(sum(inst))
    n, k = 333, 1024
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(112, 140, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    dec = oracle.dequantize(packed, scales)
    for m in (33, 77):
        cols = rng.choice(k, m, replace=False)
        x = np.zeros((m, k), np.float32)
        x[np.arange(m), cols] = 1.0
        xts = (mx4.BF16,) if inst in GEMM_BF16_ONLY else (mx4.BF16, mx4.F32)
        for xt in xts:
            xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16) if xt == mx4.BF16 else x)
            yb = ctx.buffer(m * n * 4)
            assert ctx.gemm_config(xb, xt, m, w, yb, wm, wn, tm, tn, ks) == 0, mx4.last_error()
            got = yb.download(np.float32).reshape(m, n)
            assert np.array_equal(got, dec[:, cols].T), f"identity m={m} xt={xt}"
        if inst in GEMM_BF16_ONLY:
            xb = ctx.to_device(x)
            assert ctx.gemm_config(xb, mx4.F32, m, w, ctx.buffer(m * n * 4), wm, wn, tm, tn, ks) == mx4.ERR_UNSUPPORTED
        xr = oracle.bf16_to_f32(oracle.synth_bf16(1200 + m, 1.0, m * k)).reshape(m, k)
        for xt in xts:
            xin = xr if xt == mx4.BF16 else (xr + rng.standard_normal(xr.shape).astype(np.float32) * 1e-3)
            ref = oracle.matmul(xin, packed.reshape(-1), scales.reshape(-1))
            xb = ctx.to_device((f32_bits(xin) >> 16).astype(np.uint16) if xt == mx4.BF16 else xin)
            yb = ctx.buffer(m * n * 4)
            assert ctx.gemm_config(xb, xt, m, w, yb, wm, wn, tm, tn, ks) == 0, mx4.last_error()
            got = yb.download(np.float32).reshape(m, n)
            assert_close(got, ref, f"gemm {inst} ks={ks} m={m} xt={xt}", scaled=True)
            assert ctx.gemm_config(xb, xt, m, w, yb, wm, wn, tm, tn, ks) == 0
            assert np.array_equal(yb.download(np.float32).reshape(m, n), got), "repeat"
    w.release()


@pytest.mark.parametrize("name", ["q", "gate", "down"])
def test_gemm_auto_8b_shapes(mx4, ctx, oracle, name):
    """AUTO at M = 33, 128, 384, 512 and 768 token rows on the Qwen3-8B q,
    gate and down weights (the drop-in's path for a prompt;
    engine/src/gpu.rs:510-514) takes the exact tiled GEMM, with the tile the
    round-time estimate picks (64x64 with K split, 64x128, 64x256 and 128x192
    among these): sampled token rows x weight rows against the oracle, bf16
    and f32 activations."""
    n, k = QWEN8[name]
    rng = np.random.default_rng(91)
    w = ctx.synth_weight(500 + list(QWEN8).index(name), n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    cols = _sample_rows(n, 64, rng)
    for m in (33, 128, 384, 512, 768):
        say(f"gemm AUTO 8B {name} m={m}")
        x = oracle.bf16_to_f32(oracle.synth_bf16(510 + m, 1.0, m * k)).reshape(m, k)
        rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 14, replace=False)]))
        for xt in (mx4.BF16, mx4.F32):
            xin = x if xt == mx4.BF16 else (x + rng.standard_normal(x.shape).astype(np.float32) * 1e-3)
            ref = np.concatenate([oracle.matmul_rows(xin[rows], packed.reshape(-1), scales.reshape(-1), int(c),
                                                     int(c) + 1) for c in cols], axis=1)
            y = run_matmul(mx4, ctx, xin, w, mx4.PATH_AUTO, xt)
            assert np.all(np.isfinite(y))
            assert_close(y[np.ix_(rows, cols)], ref, f"gemm AUTO {name} m={m} xt={xt}")
    w.release()


def test_gemm_rejects_and_falls_back(mx4, ctx, oracle):
    """K not a multiple of 128 or scale bytes outside 2..252: AUTO runs the
    exact generic kernel (still exact), the explicit GEMM path is refused."""
    rng = np.random.default_rng(3)
    m, n, k = 40, 50, 160
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(118, 130, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = oracle.matmul(x, packed.reshape(-1), scales.reshape(-1))
    assert_close(run_matmul(mx4, ctx, x, w, mx4.PATH_AUTO), ref, "K=160 AUTO", scaled=True)
    with pytest.raises(mx4.Mx4Error, match="K % 128"):
        run_matmul(mx4, ctx, x, w, mx4.PATH_GEMM)
    k2 = 256
    packed2 = rng.integers(0, 256, (n, k2 // 2), dtype=np.uint8)
    scales2 = rng.integers(118, 130, (n, k2 // 32), dtype=np.uint8)
    scales2[7, 3] = 1
    w2 = ctx.upload_weight(packed2, scales2, n, k2)
    x2 = rng.standard_normal((m, k2)).astype(np.float32)
    ref2 = oracle.matmul(x2, packed2.reshape(-1), scales2.reshape(-1))
    assert_close(run_matmul(mx4, ctx, x2, w2, mx4.PATH_AUTO), ref2, "scale 1 AUTO", scaled=True)
    with pytest.raises(mx4.Mx4Error, match="2..252"):
        run_matmul(mx4, ctx, x2, w2, mx4.PATH_GEMM)
    yb = ctx.buffer(m * n * 4)
    xb = ctx.to_device(x2)
    assert ctx.gemm_config(xb, mx4.F32, m, w2, yb, 3, 3, 1, 1) == mx4.ERR_UNSUPPORTED
    # a K split must cut K into whole 128-element stages
    xb3 = ctx.to_device(rng.standard_normal((m, 384)).astype(np.float32))
    w3 = ctx.synth_weight(7, n, 384, 0.02)
    assert ctx.gemm_config(xb3, mx4.F32, m, w3, yb, 2, 2, 1, 1, 2) == mx4.ERR_UNSUPPORTED
    assert ctx.gemm_config(xb3, mx4.F32, m, w3, yb, 2, 2, 1, 1, 3) == 0
    w3.release()
    w.release()
    w2.release()


def _prefill_ref(oracle, x, packed, scales, act):
    """The oracle on requantized activations: dequant(requant(x)) . dequant(W)^T."""
    if act == "mxfp4":
        xq, xs = oracle.quantize(x)
        xd = oracle.dequantize(xq, xs)
    else:
        xq, xs = oracle.quantize_fp8(x)
        xd = oracle.dequantize_fp8(xq, xs)
    return oracle.matmul(xd, packed.reshape(-1), scales.reshape(-1)), xd


def _run_prefill(mx4, ctx, x, w, act, xtype):
    m, k = x.shape
    if xtype == mx4.BF16:
        xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    else:
        xb = ctx.to_device(np.ascontiguousarray(x, np.float32))
    yb = ctx.buffer(m * w.rows * 4)
    ctx.matmul_prefill(xb, xtype, m, w, mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8, yb)
    return yb.download(np.float32).reshape(m, w.rows)


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
def test_prefill_identity_is_exact(mx4, ctx, oracle, act):
    """One-hot activations requantize exactly (1.0 -> code 4.0 at scale 2^-2, or
    E4M3 1.0), so the block-scaled MFMA must return the decoded weights bit for bit:
    pins the matrix core's E2M1 decode, the per-lane E8M0 scales and the output layout."""
    rng = np.random.default_rng(31)
    n, k, m = 64, 512, 64
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(100, 150, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    cols = rng.choice(k, m, replace=False)
    x = np.zeros((m, k), np.float32)
    x[np.arange(m), cols] = 1.0
    y = _run_prefill(mx4, ctx, x, w, act, mx4.F32)
    dec = oracle.dequantize(packed, scales)
    assert np.array_equal(y, dec[:, cols].T)


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("m,n,k", [(1, 32, 256), (7, 200, 512), (64, 128, 1024), (130, 96, 256), (256, 256, 4096),
                                   (70, 8256, 512), (33, 64, 12288), (1, 300, 4096), (33, 4100, 4096),
                                   (5, 16400, 4096)])
def test_prefill_matches_oracle_on_requantized_x(mx4, ctx, oracle, act, m, n, k):
    rng = np.random.default_rng(m * 7 + n)
    w = ctx.synth_weight(50 + m, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    x = oracle.bf16_to_f32(oracle.synth_bf16(60 + m, 1.0, m * k)).reshape(m, k)
    ref, _ = _prefill_ref(oracle, x, packed, scales, act)
    for xtype in (mx4.BF16, mx4.F32):
        y = _run_prefill(mx4, ctx, x, w, act, xtype)
        assert_close(y, ref, f"prefill {act} m={m} n={n} k={k} xtype={xtype}")


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
def test_prefill_mx_entry_matches_prefill(mx4, ctx, oracle, act):
    """mx4_matmul_mx takes row-major requantized activations (what mx4_quantize
    writes) and rearranges them for the matrix core itself: same bits as the
    fused requantize + GEMM of mx4_matmul_prefill."""
    m, n, k = 45, 160, 1024
    w = ctx.synth_weight(71, n, k, 0.02)
    x = oracle.bf16_to_f32(oracle.synth_bf16(72, 1.0, m * k)).reshape(m, k)
    y_ref = _run_prefill(mx4, ctx, x, w, act, mx4.F32)
    xb = ctx.to_device(np.ascontiguousarray(x, np.float32))
    fp8 = act == "mxfp8"
    xq = ctx.buffer(m * k if fp8 else m * k // 2)
    xs = ctx.buffer(m * k // 32)
    (ctx.quantize_fp8 if fp8 else ctx.quantize)(xb, mx4.F32, m, k, xq, xs)
    yb = ctx.buffer(m * n * 4)
    ctx.matmul_mx(xq, xs, mx4.ACT_MXFP8 if fp8 else mx4.ACT_MXFP4, m, w, yb)
    assert np.array_equal(yb.download(np.float32).reshape(m, n), y_ref)


def _to_fragments(codes, scales, fp8):
    """Row-major requantized activations -> the matrix-core fragment order
    (rows padded with zeros to a multiple of 32)."""
    r = codes.shape[0]
    g = (r + 31) // 32
    cp = np.zeros((g * 32, codes.shape[1]), np.uint8)
    cp[:r] = codes
    sp = np.zeros((g * 32, scales.shape[1]), np.uint8)
    sp[:r] = scales
    nq = scales.shape[1] // 8
    if fp8:
        nk = codes.shape[1] // 64   # byte 32 p + 16 h + b of a k-step -> [g, kk, p, h, r32, b]
        frag = cp.reshape(g, 32, nk, 2, 2, 16).transpose(0, 2, 3, 4, 1, 5)
    else:
        nk = codes.shape[1] // 32   # byte 16 h + b of a k-step -> [g, kk, h, r32, b]
        frag = cp.reshape(g, 32, nk, 2, 16).transpose(0, 2, 3, 1, 4)
    sfrag = sp.reshape(g, 32, nq, 4, 2).transpose(0, 2, 4, 1, 3)  # block 8q + 2u + h -> [g, q, h, r32, u]
    return frag.reshape(-1), sfrag.reshape(-1)


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("xtype", ["bf16", "f32"])
@pytest.mark.parametrize("k", [768, 8448])
def test_prefill_quantize_fragments_bit_exact(mx4, ctx, oracle, act, xtype, k):
    """mx4_prefill_quantize = the oracle's quantizer (python/quantize_mxfp4.py:18-39,
    or the E4M3 rule) permuted into the fragment order, byte for byte, with the
    padding rows of the last group zero; ragged rows, exact midpoints, signed zeros.
    K = 768 takes the one-k-step workgroups, K = 8448 (33 scale quads) the
    whole-quad ones."""
    rng = np.random.default_rng(17)
    m = 45
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[3, :64] = (rng.integers(-24, 25, 64) * 0.25).astype(np.float32)
    x[5, :32] = -0.0
    x[7, 32:64] = rng.standard_normal(32).astype(np.float32) * 1e-38
    if xtype == "bf16":
        bits = (f32_bits(x) >> 16).astype(np.uint16)
        x = oracle.bf16_to_f32(bits).reshape(m, k)
        xb, t = ctx.to_device(bits), mx4.BF16
    else:
        xb, t = ctx.to_device(x), mx4.F32
    fp8 = act == "mxfp8"
    code = mx4.ACT_MXFP8 if fp8 else mx4.ACT_MXFP4
    codes, sc = ctx.prefill_act_buffers(m, k, code)
    codes.upload(np.full(codes.nbytes, 0xA5, np.uint8))
    sc.upload(np.full(sc.nbytes, 0xA5, np.uint8))
    ctx.prefill_quantize(xb, t, m, k, code, codes, sc)
    want_c, want_s = (oracle.quantize_fp8 if fp8 else oracle.quantize)(x)
    frag, sfrag = _to_fragments(want_c, want_s, fp8)
    assert np.array_equal(codes.download(np.uint8), frag)
    assert np.array_equal(sc.download(np.uint8), sfrag)


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("k", [512, 8448])
def test_prefill_non_finite_activations_give_nan_rows(mx4, ctx, oracle, act, k):
    """A token row holding inf or NaN: the reference's sums over it are inf or
    NaN (engine/src/lib.rs:240-266); requantized here, its blocks carry the E8M0
    NaN scale, so every output of that row is NaN. The other rows are unaffected.
    (K = 8448: the requantizer's whole-quad workgroups, the last column too.)"""
    m, n = 40, 96
    w = ctx.synth_weight(33, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    x = oracle.bf16_to_f32(oracle.synth_bf16(34, 1.0, m * k)).reshape(m, k)
    x[3, 100] = np.inf
    x[17, 5] = np.nan
    x[20, k - 1] = -np.inf
    y = _run_prefill(mx4, ctx, x, w, act, mx4.F32)
    assert np.all(np.isnan(y[3])) and np.all(np.isnan(y[17])) and np.all(np.isnan(y[20]))
    ok = np.setdiff1d(np.arange(m), [3, 17, 20])
    ref, _ = _prefill_ref(oracle, x[ok], packed, scales, act)
    assert_close(y[ok], ref, f"prefill {act} finite rows")


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
def test_prefill_quantize_once_matmul_many(mx4, ctx, oracle, act):
    """Requantize x once in the matrix-core layout and reuse it for two weights
    (q|k|v style): each product equals the fused mx4_matmul_prefill bit for bit."""
    m, k = 77, 2048
    code = mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8
    x = oracle.bf16_to_f32(oracle.synth_bf16(91, 1.0, m * k)).reshape(m, k)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    codes, scales = ctx.prefill_act_buffers(m, k, code)
    ctx.prefill_quantize(xb, mx4.BF16, m, k, code, codes, scales)
    for seed, n in ((92, 320), (93, 96)):
        w = ctx.synth_weight(seed, n, k, 0.02)
        yb = ctx.buffer(m * n * 4)
        ctx.prefill_matmul(codes, scales, code, m, w, yb)
        assert np.array_equal(yb.download(np.float32).reshape(m, n), _run_prefill(mx4, ctx, x, w, act, mx4.BF16))


PREFILL_INSTANCES = ([(4096, t) for t in ((128, 192, 1), (128, 128, 1), (64, 128, 2), (128, 192, 2), (128, 64, 4),
                                            (64, 128, 4), (128, 96, 4), (128, 128, 4))] +
                     [(12288, t) for t in ((128, 128, 1), (64, 128, 2), (128, 192, 2), (128, 64, 4), (64, 128, 4),
                                           (128, 96, 4), (128, 128, 4))] +
                     [(1536, t) for t in ((128, 192, 1), (128, 128, 1), (64, 128, 2), (128, 192, 2))] +
                     [(2048, t) for t in ((128, 64, 4), (64, 128, 4), (128, 96, 4), (128, 128, 4))] +
                     [(1280, (128, 128, 1)), (768, (128, 128, 1))])


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("k,tile", PREFILL_INSTANCES, ids=[f"k{k}-{t[0]}x{t[1]}-ks{t[2]}" for k, t in PREFILL_INSTANCES])
def test_prefill_instances_match_oracle(mx4, ctx, oracle, act, k, tile):
    """Every prefill instance reachable through mx4_prefill_config (workgroup
    tile, K halves inside the workgroup; unrolled and loop forms) on ragged m
    and n against the oracle on dequant(requant(x)); twice, bitwise equal."""
    tm, tn, ks = tile
    m, n = (70, 300) if k <= 4096 else (40, 260)
    code = mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8
    w = ctx.synth_weight(500 + tm + tn + ks, n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    x = oracle.bf16_to_f32(oracle.synth_bf16(600 + k // 256, 1.0, m * k)).reshape(m, k)
    ref, _ = _prefill_ref(oracle, x, packed, scales, act)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    codes, sc = ctx.prefill_act_buffers(m, k, code)
    ctx.prefill_quantize(xb, mx4.BF16, m, k, code, codes, sc)
    yb = ctx.buffer(m * n * 4)
    outs = []
    for _ in range(2):
        yb.upload(np.full(m * n, np.nan, np.float32))
        assert ctx.prefill_config(codes, sc, code, m, w, yb, tm, tn, ks) == 0, mx4.last_error()
        outs.append(yb.download(np.float32).reshape(m, n))
    assert_close(outs[0], ref, f"prefill instance {tile} k={k} {act}")
    assert np.array_equal(outs[0], outs[1])


# Workgroup-shared prefill instances: tile -> waves along M x N and MFMA tiles
# per wave along M x N; split_k code 256 P + 128 (H - 1) + 16 U + D (K in H
# halves of their own waves, stages of U k-steps, ring of D; P = 1: the two
# halves in ping-pong).
LDS_TILES = {(128, 192): (2, 2, 2, 3), (128, 128): (2, 2, 2, 2), (64, 128): (2, 2, 1, 2), (128, 64): (2, 2, 2, 1),
             (64, 256): (1, 4, 2, 2), (128, 96): (4, 1, 1, 3), (64, 192): (2, 2, 1, 3), (64, 64): (2, 2, 1, 1)}
PP_CODES = (384 + 16 * 4 + 2, 384 + 16 * 4 + 3, 384 + 16 * 2 + 3, 384 + 16 * 2 + 4)
LDS_CODES = (16 * 4 + 2, 16 * 4 + 3, 16 * 2 + 3, 16 * 2 + 4, 16 * 2 + 5, 16 * 2 + 8, 16 * 4 + 5,
             128 + 16 * 4 + 2, 128 + 16 * 2 + 3, 128 + 16 * 2 + 4, 128 + 16 * 2 + 8) + PP_CODES


def code_name(c):
    """h<H>u<U>d<D>, with a trailing pp for the ping-pong schedule."""
    return f"h{2 if c & 128 else 1}u{c % 128 // 16}d{c % 16}" + ("pp" if c >= 256 else "")


def lds_depth(fp8, tile, code, k):
    """The ring depth the library compiles for (tile, split_k code) at K, or
    None: the kernel's limits (whole fragments per wave and stage, one scale
    piece per wave, waits within vmcnt, the rings -- and with two K halves the
    hand-over of the second half's tile -- within 160 KiB of LDS, each K half
    on whole scale quads), a ring that does not fit cut to the deepest that
    does (not below 2); ping-pong only with two K halves and (U, D) = (4, 2),
    (4, 3), (2, 3) or (2, 4)."""
    h, u, d = (2 if code & 128 else 1), (code % 128) // 16, code % 16
    if code >= 256 and (code >= 512 or h != 2 or (u, d) not in ((4, 2), (4, 3), (2, 3), (2, 4))):
        return None
    if k % (256 * h) != 0:
        return None
    wm, wn, tm, tn = LDS_TILES[tile]
    nw, ga, gb, afk = wm * wn, wm * tm, wn * tn, 2 if fp8 else 1
    frags = u * (ga * afk + gb)
    stage = u * ga * afk * 1024 + u * gb * 1024 + nw * 1024
    red = nw * tm * tn * 16 * 64 * 4 if h == 2 else 0

    def ok(dd):
        return (frags % nw == 0 and (ga + 3) // 4 + (gb + 3) // 4 <= nw and 2 <= dd <= 8
                and (dd - 2) * (frags // nw + 1) <= 63 and max(h * dd * stage, red) <= 160 * 1024)
    # (U, D) = (4, 2) is compiled as asked; the other codes are cut to fit
    if (u, d) == (4, 2):
        return d if ok(d) else None
    while d > 2 and not ok(d):
        d -= 1
    return d if ok(d) else None


LDS_CASES = ([(4096, t, c) for t in LDS_TILES for c in LDS_CODES] +
             [(k, t, c) for k in (256, 1280) for t in LDS_TILES for c in (16 * 4 + 2, 16 * 2 + 4)] +
             [(k, t, c) for k in (1536, 1280) for t in LDS_TILES
              for c in (128 + 16 * 4 + 2, 128 + 16 * 2 + 4, 384 + 16 * 4 + 2, 384 + 16 * 2 + 4)])


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("k,tile,code", LDS_CASES,
                         ids=[f"k{k}-{t[0]}x{t[1]}-{code_name(c)}" for k, t, c in LDS_CASES])
def test_prefill_shared_instances_match_oracle(mx4, ctx, oracle, act, k, tile, code):
    """Every workgroup-shared prefill instance reachable through
    mx4_prefill_config is compiled exactly where the kernel's limits allow it;
    each one, on ragged m and n (partial row groups and partial workgroup
    tiles), and at K = 256 / 1280 (fewer stages than the ring, an odd number of
    scale quads; with two K halves K = 1536 / 1280: three quads per half, or
    halves off the quad grid, which the library refuses), matches the oracle on
    dequant(requant(x)), twice bitwise equal."""
    fp8 = act == "mxfp8"
    h, u = (2 if code & 128 else 1), code % 128 // 16
    depth = lds_depth(fp8, tile, code, k)
    m, n = 70, 300
    acode = mx4.ACT_MXFP8 if fp8 else mx4.ACT_MXFP4
    w = ctx.synth_weight(800 + k // 256, n, k, 0.02)
    codes, sc = ctx.prefill_act_buffers(m, k, acode)
    x = oracle.bf16_to_f32(oracle.synth_bf16(810 + k // 256, 1.0, m * k)).reshape(m, k)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    ctx.prefill_quantize(xb, mx4.BF16, m, k, acode, codes, sc)
    yb = ctx.buffer(m * n * 4)
    status = ctx.prefill_config(codes, sc, acode, m, w, yb, tile[0], tile[1], code)
    if depth is None:
        assert status == mx4.ERR_UNSUPPORTED
        return
    assert status == 0, mx4.last_error()
    say(f"shared prefill {act} k={k} tile={tile} H={h} U={u} D={depth} pp={code >= 256}")
    packed, scales = ctx.download_weight(w)
    ref, _ = _prefill_ref(oracle, x, packed, scales, act)
    outs = []
    for _ in range(2):
        yb.upload(np.full(m * n, np.nan, np.float32))
        assert ctx.prefill_config(codes, sc, acode, m, w, yb, tile[0], tile[1], code) == 0, mx4.last_error()
        outs.append(yb.download(np.float32).reshape(m, n))
    assert_close(outs[0], ref, f"shared prefill {tile} H={h} U={u} D={depth} k={k} {act}")
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("tile", list(LDS_TILES), ids=[f"{t[0]}x{t[1]}" for t in LDS_TILES])
def test_prefill_shared_identity_is_exact(mx4, ctx, oracle, act, tile):
    """One-hot activations through each workgroup-shared tile (stages of 4 and
    of 2 k-steps, one ring or two K halves): the decoded weights bit for bit,
    which pins the LDS placement of every fragment and scale piece, the op_sel
    of each k-step within its quad, each half's K range and the output
    layout."""
    rng = np.random.default_rng(37)
    n, k, m = 200, 1024, 96
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(100, 150, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    cols = rng.choice(k, m, replace=False)
    x = np.zeros((m, k), np.float32)
    x[np.arange(m), cols] = 1.0
    acode = mx4.ACT_MXFP8 if act == "mxfp8" else mx4.ACT_MXFP4
    codes, sc = ctx.prefill_act_buffers(m, k, acode)
    ctx.prefill_quantize(ctx.to_device(np.ascontiguousarray(x, np.float32)), mx4.F32, m, k, acode, codes, sc)
    dec = oracle.dequantize(packed, scales)
    yb = ctx.buffer(m * n * 4)
    ran = 0
    for code in (16 * 4 + 2, 16 * 2 + 3, 128 + 16 * 4 + 2, 128 + 16 * 2 + 3, 384 + 16 * 4 + 2, 384 + 16 * 2 + 3):
        if lds_depth(act == "mxfp8", tile, code, k) is None:
            continue
        yb.upload(np.full(m * n, np.nan, np.float32))
        assert ctx.prefill_config(codes, sc, acode, m, w, yb, tile[0], tile[1], code) == 0, mx4.last_error()
        assert np.array_equal(yb.download(np.float32).reshape(m, n), dec[:, cols].T), (tile, code)
        ran += 1
    assert ran >= 1


PP_CASES = [(k, t, c) for k in (4096, 1536) for t in LDS_TILES for c in PP_CODES]


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("k,tile,code", PP_CASES, ids=[f"k{k}-{t[0]}x{t[1]}-{code_name(c)}" for k, t, c in PP_CASES])
def test_prefill_ping_pong_equals_halves(mx4, ctx, oracle, act, k, tile, code):
    """The ping-pong schedule changes when each K half's waves read LDS and
    issue MFMAs, not the arithmetic: its output is the same bits as the two K
    halves without it (same tile, stage and ring), on ragged m and n, and
    repeated calls agree."""
    fp8 = act == "mxfp8"
    depth = lds_depth(fp8, tile, code, k)
    if depth is None:
        return
    assert lds_depth(fp8, tile, code - 256, k) == depth
    m, n = 100, 250
    acode = mx4.ACT_MXFP8 if fp8 else mx4.ACT_MXFP4
    w = ctx.synth_weight(830 + k // 256, n, k, 0.02)
    x = oracle.bf16_to_f32(oracle.synth_bf16(840 + k // 256, 1.0, m * k)).reshape(m, k)
    codes, sc = ctx.prefill_act_buffers(m, k, acode)
    ctx.prefill_quantize(ctx.to_device((f32_bits(x) >> 16).astype(np.uint16)), mx4.BF16, m, k, acode, codes, sc)
    yb = ctx.buffer(m * n * 4)
    outs = []
    for c in (code - 256, code, code):
        yb.upload(np.full(m * n, np.nan, np.float32))
        assert ctx.prefill_config(codes, sc, acode, m, w, yb, tile[0], tile[1], c) == 0, mx4.last_error()
        outs.append(yb.download(np.float32))
    assert np.all(np.isfinite(outs[0]))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), (tile, code_name(code))
    assert np.array_equal(outs[1].view(np.uint32), outs[2].view(np.uint32))


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
def test_prefill_8b_defaults_repeat_bit_for_bit(mx4, ctx, oracle, act):
    """The default prefill launches at the Qwen3-8B shapes (M = 512: q|k|v and
    gate|up grouped, o/q, gate, down; ping-pong and one-ring workgroup-shared
    kernels) give the same bits on 12 calls in a row, eager and replayed from a
    recorded pass: every LDS ring slot is refilled only after all its readers
    are done, whatever the timing."""
    m = 512
    code = mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8
    groups = [["q", "k", "v"], ["q"], ["gate"], ["gate", "up"], ["down"]]
    for gi, names in enumerate(groups):
        k = QWEN8[names[0]][1]
        ns = [QWEN8[nm][0] for nm in names]
        say(f"prefill 8B defaults repeat {act} {'|'.join(names)}")
        ws = [ctx.synth_weight(450 + 10 * gi + i, n, k, 0.02) for i, n in enumerate(ns)]
        xb = ctx.to_device(oracle.synth_bf16(460 + gi, 1.0, m * k))
        codes, sc = ctx.prefill_act_buffers(m, k, code)
        ctx.prefill_quantize(xb, mx4.BF16, m, k, code, codes, sc)
        ys = [ctx.buffer(m * n * 4) for n in ns]

        def run():
            if len(ws) == 1:
                ctx.prefill_matmul(codes, sc, code, m, ws[0], ys[0])
            else:
                ctx.prefill_matmul_group(codes, sc, code, m, ws, ys)

        def grab():
            return np.concatenate([y.download(np.float32) for y in ys]).view(np.uint32)

        run()
        first = grab()
        assert np.all(np.isfinite(first.view(np.float32)))
        for _ in range(5):
            for y, n in zip(ys, ns):
                y.upload(np.full(m * n, np.nan, np.float32))
            run()
            assert np.array_equal(grab(), first), names
        p = ctx.record(lambda: [run() for _ in range(6)])
        for _ in range(2):
            for y, n in zip(ys, ns):
                y.upload(np.full(m * n, np.nan, np.float32))
            p.launch()
            assert np.array_equal(grab(), first), names
        p.release()
        for w in ws:
            w.release()


GROUP_TILES = [(0, 0, 0), (128, 192, 1), (128, 128, 1), (64, 128, 2), (128, 192, 2), (128, 64, 4), (64, 128, 4),
               (64, 128, 16 * 2 + 4), (128, 192, 16 * 2 + 3), (64, 128, 16 * 4 + 2),
               (128, 128, 384 + 16 * 4 + 2), (128, 192, 384 + 16 * 2 + 3)]


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
def test_prefill_group_equals_individual(mx4, ctx, oracle, act):
    """One grouped launch over three weights of the same K (ragged rows, as
    q|k|v) gives each weight's output bit for bit as the same instance run on
    that weight alone, for every instance and the default; the default group
    also matches the oracle on dequant(requant(x))."""
    m, k = 70, 2048
    ns = (300, 96, 160)
    code = mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8
    ws = [ctx.synth_weight(700 + i, n, k, 0.02) for i, n in enumerate(ns)]
    x = oracle.bf16_to_f32(oracle.synth_bf16(710, 1.0, m * k)).reshape(m, k)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    codes, sc = ctx.prefill_act_buffers(m, k, code)
    ctx.prefill_quantize(xb, mx4.BF16, m, k, code, codes, sc)
    ys = [ctx.buffer(m * n * 4) for n in ns]
    y1 = ctx.buffer(max(ns) * m * 4)
    for tile in GROUP_TILES:
        if tile[2] >= 16 and lds_depth(act == "mxfp8", tile[:2], tile[2], k) is None:
            continue  # e.g. stages of 4 on 128 x 128 MX-FP8 tiles in two rings outgrow the LDS
        say(f"prefill group {act} tile {tile}")
        for y, n in zip(ys, ns):
            y.upload(np.full(m * n, np.nan, np.float32))
        assert ctx.prefill_group_config(codes, sc, code, m, ws, ys, *tile) == 0, mx4.last_error()
        for w, y, n in zip(ws, ys, ns):
            y1.upload(np.full(m * max(ns), np.nan, np.float32))
            assert ctx.prefill_config(codes, sc, code, m, w, y1, *tile) == 0, mx4.last_error()
            alone = y1.download(np.float32)[: m * n].reshape(m, n)
            assert np.array_equal(y.download(np.float32).reshape(m, n), alone), (tile, n)
    for y, n in zip(ys, ns):
        y.upload(np.full(m * n, np.nan, np.float32))
    ctx.prefill_matmul_group(codes, sc, code, m, ws, ys)
    for w, y, n in zip(ws, ys, ns):
        packed, scales = ctx.download_weight(w)
        ref, _ = _prefill_ref(oracle, x, packed, scales, act)
        assert_close(y.download(np.float32).reshape(m, n), ref, f"prefill group {act} n={n}")


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
def test_matmul_prefill_group_requantizes_once(mx4, ctx, oracle, act):
    """mx4_matmul_prefill_group (requantize + one grouped launch) at 8B widths
    (q|k|v rows 4096 + 1024 + 1024, K = 4096, the workgroup-shared kernel's
    default there; ragged m) against the oracle, and equal to the grouped
    launch on activations requantized beforehand."""
    m, k = 40, 4096
    ns = (4096, 1024, 1024)
    code = mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8
    ws = [ctx.synth_weight(720 + i, n, k, 0.02) for i, n in enumerate(ns)]
    x = oracle.bf16_to_f32(oracle.synth_bf16(730, 1.0, m * k)).reshape(m, k)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    ys = [ctx.buffer(m * n * 4) for n in ns]
    ctx.matmul_prefill_group(xb, mx4.BF16, m, ws, code, ys)
    got = [y.download(np.float32).reshape(m, n) for y, n in zip(ys, ns)]
    codes, sc = ctx.prefill_act_buffers(m, k, code)
    ctx.prefill_quantize(xb, mx4.BF16, m, k, code, codes, sc)
    ctx.prefill_matmul_group(codes, sc, code, m, ws, ys)
    for i, (w, y, n) in enumerate(zip(ws, ys, ns)):
        assert np.array_equal(y.download(np.float32).reshape(m, n), got[i])
        packed, scales = ctx.download_weight(w)
        rows = np.arange(0, n, 7)
        ref, _ = _prefill_ref(oracle, x, packed.reshape(n, -1)[rows], scales.reshape(n, -1)[rows], act)
        assert_close(got[i][:, rows], ref, f"grouped requant + prefill {act} n={n}")


def test_prefill_group_rejects_bad_groups(mx4, ctx):
    m, k = 32, 1024
    w1, w2 = ctx.synth_weight(740, 64, k, 0.02), ctx.synth_weight(741, 64, 2048, 0.02)
    codes, sc = ctx.prefill_act_buffers(m, k, mx4.ACT_MXFP4)
    y = ctx.buffer(m * 64 * 4)
    with pytest.raises(mx4.Mx4Error, match="share K"):
        ctx.prefill_matmul_group(codes, sc, mx4.ACT_MXFP4, m, [w1, w2], [y, y])
    with pytest.raises(mx4.Mx4Error, match="1 to 4"):
        ctx.prefill_matmul_group(codes, sc, mx4.ACT_MXFP4, m, [w1] * 5, [y] * 5)
    with pytest.raises(mx4.Mx4Error, match="1 to 4"):
        ctx.prefill_matmul_group(codes, sc, mx4.ACT_MXFP4, m, [], [])


def test_prefill_config_rejects_unknown_instance(mx4, ctx):
    m, n, k = 64, 256, 4096
    w = ctx.synth_weight(7, n, k, 0.02)
    codes, sc = ctx.prefill_act_buffers(m, k, mx4.ACT_MXFP4)
    yb = ctx.buffer(m * n * 4)
    assert ctx.prefill_config(codes, sc, mx4.ACT_MXFP4, m, w, yb, 96, 256, 1) == mx4.ERR_UNSUPPORTED
    assert ctx.prefill_config(codes, sc, mx4.ACT_MXFP4, m, w, yb, 64, 64, 4) == mx4.ERR_UNSUPPORTED
    # workgroup-shared kernel: a tile it does not compile, a stage of 3 k-steps, a ring of 6
    assert ctx.prefill_config(codes, sc, mx4.ACT_MXFP4, m, w, yb, 96, 64, 16 * 4 + 2) == mx4.ERR_UNSUPPORTED
    assert ctx.prefill_config(codes, sc, mx4.ACT_MXFP4, m, w, yb, 64, 128, 16 * 3 + 3) == mx4.ERR_UNSUPPORTED
    assert ctx.prefill_config(codes, sc, mx4.ACT_MXFP4, m, w, yb, 64, 128, 16 * 2 + 6) == mx4.ERR_UNSUPPORTED
    # ping-pong: without two K halves, with a stage and ring it does not
    # compile, and codes past it
    assert ctx.prefill_config(codes, sc, mx4.ACT_MXFP4, m, w, yb, 64, 128, 256 + 16 * 2 + 3) == mx4.ERR_UNSUPPORTED
    assert ctx.prefill_config(codes, sc, mx4.ACT_MXFP4, m, w, yb, 64, 128, 384 + 16 * 2 + 5) == mx4.ERR_UNSUPPORTED
    assert ctx.prefill_config(codes, sc, mx4.ACT_MXFP4, m, w, yb, 64, 128, 512 + 128 + 16 * 2 + 3) == mx4.ERR_UNSUPPORTED
    # K quarters must start on whole scale quads (K % 1024 == 0)
    w2 = ctx.synth_weight(8, n, 1536, 0.02)
    codes2, sc2 = ctx.prefill_act_buffers(m, 1536, mx4.ACT_MXFP4)
    assert ctx.prefill_config(codes2, sc2, mx4.ACT_MXFP4, m, w2, yb, 128, 64, 4) == mx4.ERR_UNSUPPORTED


def test_prefill_recorded_pass_after_prepare(mx4, ctx, oracle):
    """The matrix-core copy of a weight is built outside the pass
    (mx4_weight_prepare_prefill) and the workspace reserved; every replay of the
    recorded prefill equals the eager result. Without the prepare the recording
    fails with an error instead of allocating."""
    m, n, k = 96, 256, 2048
    w = ctx.synth_weight(81, n, k, 0.02)
    x = oracle.bf16_to_f32(oracle.synth_bf16(82, 1.0, m * k)).reshape(m, k)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    yb = ctx.buffer(m * n * 4)
    w2 = ctx.synth_weight(83, n, k, 0.02)
    ctx.reserve_prefill(m, k)
    with pytest.raises(mx4.Mx4Error, match="prepare"):
        ctx.record(lambda: ctx.matmul_prefill(xb, mx4.BF16, m, w2, mx4.ACT_MXFP4, yb))
    w.prepare_prefill()
    eager = _run_prefill(mx4, ctx, x, w, "mxfp4", mx4.BF16)
    p = ctx.record(lambda: ctx.matmul_prefill(xb, mx4.BF16, m, w, mx4.ACT_MXFP4, yb))
    for _ in range(3):
        yb.upload(np.zeros(m * n, np.float32))
        p.launch()
        ctx.synchronize()
        assert np.array_equal(yb.download(np.float32).reshape(m, n), eager)
    p.release()


def _requant(oracle, x, act):
    if act == "mxfp4":
        return oracle.dequantize(*oracle.quantize(x))
    return oracle.dequantize_fp8(*oracle.quantize_fp8(x))


def _sampled_ref(oracle, xd, packed, scales, cols):
    return np.concatenate([oracle.matmul_rows(xd, packed.reshape(-1), scales.reshape(-1), int(c), int(c) + 1)
                           for c in cols], axis=1)


def test_recorded_pass_survives_workspace_growth(mx4, ctx, oracle):
    """A recorded prefill reads the context's requantization workspace. A later
    eager call that needs a larger workspace must not free the buffer the pass
    holds: every replay afterwards still equals the eager result, and the
    larger call itself is correct."""
    m, n, k = 64, 256, 2048
    w = ctx.synth_weight(85, n, k, 0.02)
    w.prepare_prefill()
    x = oracle.bf16_to_f32(oracle.synth_bf16(86, 1.0, m * k)).reshape(m, k)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    yb = ctx.buffer(m * n * 4)
    ctx.reserve_prefill(m, k)
    eager = _run_prefill(mx4, ctx, x, w, "mxfp4", mx4.BF16)
    p = ctx.record(lambda: ctx.matmul_prefill(xb, mx4.BF16, m, w, mx4.ACT_MXFP4, yb))
    # an eager prefill 16x larger than the reservation grows the workspace
    m2, k2 = 512, 8192
    w2 = ctx.synth_weight(87, 64, k2, 0.02)
    x2 = oracle.bf16_to_f32(oracle.synth_bf16(88, 1.0, m2 * k2)).reshape(m2, k2)
    y2 = _run_prefill(mx4, ctx, x2, w2, "mxfp8", mx4.BF16)
    packed2, scales2 = ctx.download_weight(w2)
    rows = np.arange(0, m2, 37)
    ref2, _ = _prefill_ref(oracle, x2[rows], packed2, scales2, "mxfp8")
    assert_close(y2[rows], ref2, "grown workspace")
    for _ in range(3):
        yb.upload(np.zeros(m * n, np.float32))
        p.launch()
        ctx.synchronize()
        assert np.array_equal(yb.download(np.float32).reshape(m, n), eager)
    p.release()
    # with no pass alive the next growth frees at once; results stay right
    y3 = _run_prefill(mx4, ctx, x, w, "mxfp4", mx4.BF16)
    assert np.array_equal(y3, eager)
    w.release()
    w2.release()


@pytest.mark.parametrize("m", [128, 256, 512, 640, 1024, 2048])
@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("name", ["q", "o", "gate", "up", "down"])
def test_prefill_8b_shapes_sampled(mx4, ctx, oracle, name, act, m):
    """Every Qwen3-8B prefill shape (q/o 4096->4096, gate/up 4096->12288,
    down 12288->4096) at 128 / 256 / 512 / 640 / 1024 / 2048 token rows, MXFP4 and
    MX-FP8 activations: 24 token rows x sampled weight rows against the oracle
    on dequant(requant(x)), through the default instance of each shape and row
    count (away from 512 rows, the tile nearest one round of the CUs; beyond
    that, 128 x 128 for q, o and down)."""
    rng = np.random.default_rng(77 + m)
    n, k = QWEN8[name]
    say(f"prefill 8B {name} {act} {m} x {k} -> {n}")
    w = ctx.synth_weight(400 + list(QWEN8).index(name), n, k, 0.02)
    packed, scales = ctx.download_weight(w)
    x = oracle.bf16_to_f32(oracle.synth_bf16(401, 1.0, m * k)).reshape(m, k)
    rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 22, replace=False)]))
    cols = _sample_rows(n, 96, rng)
    ref = _sampled_ref(oracle, _requant(oracle, x[rows], act), packed, scales, cols)
    y = _run_prefill(mx4, ctx, x, w, act, mx4.BF16)
    assert_close(y[np.ix_(rows, cols)], ref, f"prefill 8B {name} {act}")
    w.release()


def test_weight_layouts_footprint_release_and_drop(mx4, ctx, oracle):
    """Resident layouts of one weight: the stored layout and the matrix-core
    copy are reported; the copy can be released after a prefill phase and is
    rebuilt on the next call (same results); a weight that serves prefill only
    can drop its stored layout (one copy left), after which prefill results are
    unchanged and every other entry point refuses it; neither layout is freed
    while a recorded pass of the context is alive; a wrapped weight's memory is
    the caller's and cannot be dropped."""
    rng = np.random.default_rng(21)
    m, n, k = 64, 200, 2048
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(118, 130, (n, k // 32), dtype=np.uint8)
    w = ctx.upload_weight(packed, scales, n, k)
    stored, copy = w.footprint()
    assert stored == n * k // 2 + n * k // 32 and copy == 0
    x = oracle.bf16_to_f32(oracle.synth_bf16(22, 1.0, m * k)).reshape(m, k)
    y0 = _run_prefill(mx4, ctx, x, w, "mxfp4", mx4.BF16)
    stored, copy = w.footprint()
    assert copy >= n * k // 2 and copy < 1.2 * stored
    # a live recorded pass may read either layout: both frees are refused until it is released
    xb1 = ctx.to_device((f32_bits(x[:1]) >> 16).astype(np.uint16))
    yb1 = ctx.buffer(n * 4)
    p = ctx.record(lambda: ctx.matmul(xb1, mx4.BF16, 1, w, yb1))
    with pytest.raises(mx4.Mx4Error, match="release the passes first"):
        w.release_prefill()
    with pytest.raises(mx4.Mx4Error, match="release the passes first"):
        w.drop_stored()
    p.launch()
    p.release()
    assert w.footprint() == (stored, copy)
    w.release_prefill()
    assert w.footprint() == (stored, 0)
    assert np.array_equal(_run_prefill(mx4, ctx, x, w, "mxfp4", mx4.BF16), y0)
    w.drop_stored()
    assert w.footprint()[0] == 0 and w.footprint()[1] == copy
    assert np.array_equal(_run_prefill(mx4, ctx, x, w, "mxfp4", mx4.BF16), y0)
    with pytest.raises(mx4.Mx4Error, match="stored layout was dropped"):
        run_matmul(mx4, ctx, x, w, mx4.PATH_AUTO, mx4.BF16)
    with pytest.raises(mx4.Mx4Error, match="only layout"):
        w.release_prefill()
    w.release()
    w2 = ctx.synth_weight(23, n, k, 0.02)  # wrapped around a buffer the caller owns
    with pytest.raises(mx4.Mx4Error, match="belongs to the caller"):
        w2.drop_stored()
    w2.release()


@pytest.mark.parametrize("m", [1024, 2048])
@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
def test_prefill_8b_qkv_group_many_rows(mx4, ctx, oracle, act, m):
    """q|k|v beyond 768 token rows through mx4_matmul_prefill_group (MXFP4:
    128 x 128 tiles over the whole K, two workgroups per CU; MX-FP8: its
    one-ring 64 x 128 tiles) against the oracle on sampled token rows and
    weight rows of each member, and against each member's single launch."""
    rng = np.random.default_rng(79 + m)
    k = 4096
    ns = [QWEN8["q"][0], QWEN8["k"][0], QWEN8["v"][0]]
    say(f"prefill 8B q|k|v group {act} {m} rows")
    ws = [ctx.synth_weight(420 + i, n, k, 0.02) for i, n in enumerate(ns)]
    x = oracle.bf16_to_f32(oracle.synth_bf16(421 + m, 1.0, m * k)).reshape(m, k)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    code = mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8
    ys = [ctx.buffer(m * n * 4) for n in ns]
    ctx.matmul_prefill_group(xb, mx4.BF16, m, ws, code, ys)
    rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 14, replace=False)]))
    xd = _requant(oracle, x[rows], act)
    for i, (w, n) in enumerate(zip(ws, ns)):
        got = ys[i].download(np.float32).reshape(m, n)
        packed, scales = ctx.download_weight(w)
        cols = _sample_rows(n, 48, rng)
        assert_close(got[np.ix_(rows, cols)], _sampled_ref(oracle, xd, packed, scales, cols),
                     f"q|k|v group {act} m={m} weight {i}")
        single = _run_prefill(mx4, ctx, x, w, act, mx4.BF16)
        assert_close(got, single, f"q|k|v group {act} m={m} weight {i} against its single launch")
    for w in ws:
        w.release()


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
def test_prefill_8b_gate_up_group(mx4, ctx, oracle, act):
    """gate|up at M = 512 through mx4_matmul_prefill_group (engine/src/lib.rs:459-467:
    both read the same activations; one requantization, one launch) against the
    oracle on sampled rows and columns, and against the single-weight launches
    (the group runs the workgroup-shared kernel, a weight alone the
    register-direct one: only the summation order differs; bitwise equality of
    a group and its members on the same instance is tested on every instance)."""
    rng = np.random.default_rng(78)
    n, k = QWEN8["gate"]
    m = 512
    say(f"prefill 8B gate|up group {act}")
    ws = [ctx.synth_weight(410 + i, n, k, 0.02) for i in range(2)]
    x = oracle.bf16_to_f32(oracle.synth_bf16(411, 1.0, m * k)).reshape(m, k)
    xb = ctx.to_device((f32_bits(x) >> 16).astype(np.uint16))
    code = mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8
    ys = [ctx.buffer(m * n * 4) for _ in ws]
    ctx.matmul_prefill_group(xb, mx4.BF16, m, ws, code, ys)
    rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 14, replace=False)]))
    xd = _requant(oracle, x[rows], act)
    for i, w in enumerate(ws):
        got = ys[i].download(np.float32).reshape(m, n)
        packed, scales = ctx.download_weight(w)
        cols = _sample_rows(n, 64, rng)
        assert_close(got[np.ix_(rows, cols)], _sampled_ref(oracle, xd, packed, scales, cols),
                     f"gate|up group {act} weight {i}")
        single = _run_prefill(mx4, ctx, x, w, act, mx4.BF16)
        assert_close(got, single, f"gate|up group {act} weight {i} against its single launch")
    for w in ws:
        w.release()
