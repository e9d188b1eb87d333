"""mx4_matmul_prefill_noalloc, the prefill entry point that allocates nothing
(its workspace is the library's fixed per-device array), against
mx4_matmul_prefill on the same inputs through the C ABI: the same kernels, so
the outputs must be equal bit for bit. Two calls in a row, the second on a
smaller input (the workspace keeps the first call's contents), both
activation formats, bf16 and f32 activations; a recorded pass with no
workspace reserved; the size limit and the missing matrix-core copy are
reported as errors before anything is launched."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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


def _bits(x):
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _inputs(ctx, oracle, mx4, m, k, seed, xtype):
    x = oracle.bf16_to_f32(oracle.synth_bf16(seed, 1.0, m * k)).reshape(m, k)
    if xtype == mx4.F32:
        x = x + np.float32(1e-3) * oracle.bf16_to_f32(oracle.synth_bf16(seed + 1, 1.0, m * k)).reshape(m, k)
        return ctx.to_device(np.ascontiguousarray(x, np.float32))
    return ctx.to_device(_bits(x))


@pytest.mark.parametrize("act", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("xtype", ["bf16", "f32"])
def test_noalloc_equals_prefill_twice(mx4, ctx, oracle, act, xtype):
    code = mx4.ACT_MXFP4 if act == "mxfp4" else mx4.ACT_MXFP8
    xt = mx4.BF16 if xtype == "bf16" else mx4.F32
    # first call: the largest documented case (M = 512, K = 12288) on a
    # 96-row weight; second call: a smaller input (ragged m, K = 4096)
    cases = [(512, 96, 12288, 5), (37, 200, 4096, 6)]
    for i, (m, n, k, seed) in enumerate(cases):
        say(f"no-alloc prefill {act} x={xtype} call {i}: m={m} n={n} k={k}")
        w = ctx.synth_weight(900 + seed, n, k, 0.02)
        w.prepare_prefill()
        xb = _inputs(ctx, oracle, mx4, m, k, 910 + seed, xt)
        y_ref = ctx.buffer(m * n * 4)
        y_new = ctx.buffer(m * n * 4)
        y_new.upload(np.full(m * n, np.nan, np.float32))
        ctx.matmul_prefill(xb, xt, m, w, code, y_ref)
        ctx.matmul_prefill_noalloc(xb, xt, m, w, code, y_new)
        ctx.synchronize()
        want = y_ref.download(np.float32)
        got = y_new.download(np.float32)
        assert np.all(np.isfinite(want))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"call {i}"
        # and against the oracle on a few rows (dequant(requant(x)) . W^T)
        packed, scales = ctx.download_weight(w)
        xs = xb.download(np.uint16 if xt == mx4.BF16 else np.float32)
        xf = oracle.bf16_to_f32(xs) if xt == mx4.BF16 else xs
        xf = xf.reshape(m, k)[[0, m - 1]]
        xd = oracle.dequantize(*oracle.quantize(xf)) if act == "mxfp4" else oracle.dequantize_fp8(*oracle.quantize_fp8(xf))
        ref = oracle.matmul(xd, packed.reshape(-1), scales.reshape(-1))
        g2 = got.reshape(m, n)[[0, m - 1]]
        assert float(np.max(np.abs(g2 - ref)) / np.max(np.abs(ref))) <= 1e-3
        w.release()


def test_noalloc_records_into_a_pass_without_reservation(mx4, ctx, oracle):
    """Recording needs no workspace reservation: every replay equals the eager
    call (mx4_matmul_prefill would need mx4_reserve_prefill first)."""
    m, n, k = 200, 160, 4096
    w = ctx.synth_weight(950, n, k, 0.02)
    w.prepare_prefill()
    xb = _inputs(ctx, oracle, mx4, m, k, 951, mx4.BF16)
    y = ctx.buffer(m * n * 4)
    ctx.matmul_prefill_noalloc(xb, mx4.BF16, m, w, mx4.ACT_MXFP8, y)
    ctx.synchronize()
    eager = y.download(np.float32)
    p = ctx.record(lambda: ctx.matmul_prefill_noalloc(xb, mx4.BF16, m, w, mx4.ACT_MXFP8, y))
    for rep in range(3):
        y.upload(np.zeros(m * n, np.float32))
        p.launch()
        ctx.synchronize()
        assert np.array_equal(y.download(np.float32), eager), rep
    p.release()
    w.release()


def test_noalloc_rejects_what_it_cannot_hold(mx4, ctx):
    m, k = 1024, 12288  # MX-FP8: 12 MiB of codes, beyond the 8 MiB workspace
    w = ctx.synth_weight(960, 64, k, 0.02)
    w.prepare_prefill()
    xb = ctx.buffer(m * k * 2)
    y = ctx.buffer(m * 64 * 4)
    with pytest.raises(mx4.Mx4Error, match="no-alloc workspace holds") as e:
        ctx.matmul_prefill_noalloc(xb, mx4.BF16, m, w, mx4.ACT_MXFP8, y)
    assert e.value.status == mx4.ERR_TOO_LARGE
    w2 = ctx.synth_weight(961, 64, 4096, 0.02)  # no matrix-core copy yet
    x2 = ctx.buffer(32 * 4096 * 2)
    y2 = ctx.buffer(32 * 64 * 4)
    with pytest.raises(mx4.Mx4Error, match="mx4_weight_prepare_prefill") as e2:
        ctx.matmul_prefill_noalloc(x2, mx4.BF16, 32, w2, mx4.ACT_MXFP4, y2)
    assert e2.value.status == mx4.ERR_UNSUPPORTED
    w.release()
    w2.release()
