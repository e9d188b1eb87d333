"""The matrix-core ceiling probe (mx4_mfma_ceiling) that the prefill figures
are read against. These check the measurement, not numerics: the rate it
reports cannot exceed one MFMA per nominal issue time at the clock the waves
held on the device's own SIMDs, and the clock is a plausible shader clock for
this part (at most its 2.4 GHz peak). How close the probe comes to the issue
limit is a measurement, reported by bench.py, not asserted here."""
import sys

import pytest

pytestmark = pytest.mark.gpu

# MI355X: 256 CUs (the device reports its own count) x 4 SIMDs. Issue rates
# per SIMD (the published dense peaks at 2.4 GHz): a block-scaled FP4 x FP4
# 32x32x64 MFMA (131072 flops) every 32 cycles and its 16x16x128 form (65536
# flops) every 16, 4096 flops per cycle; FP8 x FP4 32x32x64 at half that;
# bf16 32x32x16 (32768 flops) every 32 cycles, 1024 flops per cycle.
FLOPS_PER_CYCLE_PER_SIMD = {0: 4096, 1: 4096, 2: 2048, 3: 1024}
PEAK_CLOCK_GHZ = 2.4


@pytest.fixture(scope="module")
def ctx():
    import mx4hip

    if mx4hip.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    c = mx4hip.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("shape", [0, 1, 2, 3], ids=["fp4-32x32x64", "fp4-16x16x128", "fp8xfp4-32x32x64",
                                                    "bf16-32x32x16"])
@pytest.mark.parametrize("random_codes", [True, False], ids=["random", "constant"])
def test_mfma_ceiling_is_a_physical_rate(ctx, shape, random_codes):
    pf, ghz = ctx.mfma_ceiling(shape, random_codes)
    simds = ctx.compute_units() * 4
    at_clock = FLOPS_PER_CYCLE_PER_SIMD[shape] * simds * ghz * 1e9 / 1e15
    print(f"mfma ceiling shape {shape} random {random_codes}: {pf:.2f} PF at {ghz:.3f} GHz "
          f"(issue-limited rate at that clock {at_clock:.2f} PF, {pf / at_clock:.2f} of it)", flush=True)
    sys.stdout.flush()
    # physical bounds only (a busy or partitioned device may run the probe
    # slower; bench.py reports the fraction)
    assert 0.3 < ghz <= PEAK_CLOCK_GHZ * 1.02
    assert 0 < pf <= at_clock * 1.02


def test_mfma_ceiling_rejects_bad_shape(ctx):
    import mx4hip

    with pytest.raises(mx4hip.Mx4Error, match="shape"):
        ctx.mfma_ceiling(4, True)


def test_mfma_ceiling_leaves_the_context_timer_alone(ctx):
    """The probe times itself with events of its own: a caller's
    mx4_timer_begin/end around it still measures from its own begin (the
    probe's two runs, about 0.3 ms each, fall inside)."""
    ctx.timer_begin()
    ctx.mfma_ceiling(0, True)
    ms = ctx.timer_end()
    assert ms > 0.4
