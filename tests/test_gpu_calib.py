"""The MFMA-ceiling measurement bench.py reports beside the published peak: it runs, and
its rate, clock and cycles per MFMA are consistent with each other and with the part's
limits (2.5 PFLOP/s bf16 and 5.0 POP/s int8/fp8 dense at the top clock)."""
import pytest

import bench

pytestmark = pytest.mark.gpu

# kind -> (published dense peak at the top clock, ops per MFMA): the 32x32 shapes the
# kernels use and the 16x16 shapes of the same types
PEAK = {0: (2500.0, 32768), 1: (5000.0, 65536), 2: (5000.0, 131072),
        3: (2500.0, 16384), 4: (5000.0, 32768), 5: (5000.0, 65536)}


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5])
def test_mfma_ceiling_is_consistent(kind):
    r = bench.mfma_ceiling(kind, iters=400, reps=2)
    assert r is not None, "libmoddit_calib.so missing or the measurement failed"
    peak, ops = PEAK[kind]
    assert 0.2 * peak < r["value"] <= 1.02 * peak, r
    assert 500 <= r["clock_mhz"] <= 2600, r
    # an MFMA cannot issue faster than its pass count: the published peak is 1024 SIMDs
    # x ops per MFMA / (minimum cycles per MFMA) at 2.4 GHz
    min_cycles = 1024 * ops * 2.4e9 / (peak * 1e12)
    assert r["cycles_per_mfma_per_simd"] >= 0.97 * min_cycles, (min_cycles, r)
