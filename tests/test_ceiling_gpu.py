"""The MFMA throughput probe behind bench.py --ceiling runs and reports sane
figures: zero operands reach at least 90 % of the 2.4 GHz dense peak scaled
to the clock it reports, and no mode exceeds the published peak."""

import ctypes

import pytest

from gfx906_amd.build import CEILING_LIB

pytestmark = pytest.mark.gpu

PEAK = 2516.6


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
def test_ceiling_modes(mode):
    lib = ctypes.CDLL(str(CEILING_LIB))
    lib.mfma_ceiling.restype = ctypes.c_int
    tf, ghz = ctypes.c_double(), ctypes.c_double()
    assert lib.mfma_ceiling(mode, 2000, 3, ctypes.byref(tf), ctypes.byref(ghz)) == 0
    print(f"mode {mode}: {tf.value:.1f} TFLOP/s at {ghz.value:.3f} GHz", flush=True)
    assert 0.5 < ghz.value < 3.0
    assert 0 < tf.value <= PEAK * 1.02
    if mode == 1:
        assert tf.value >= 0.9 * PEAK * ghz.value / 2.4
