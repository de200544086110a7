"""th_capture_begin / th_capture_end / th_graph_launch: a capture whose
recorded call fails its argument checks raises that error and leaves the
device stream usable (the capture is ended, its graph freed); a replay of a
q4 GEMV graph matches the eager call bit for bit."""
import numpy as np
import pytest

from tang_amd import capi

pytestmark = pytest.mark.gpu


def test_failed_capture_leaves_stream_usable(dev):
    rows, cols = 64, 256
    nib, sc16 = capi.synth_q4(5, rows, cols)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    x = dev.upload(capi.synth_normal(6, cols, 1.0, capi.BF16), capi.BF16)
    short = dev.alloc(3)
    with pytest.raises(capi.TangHipError):
        dev.capture(lambda: dev.gemm_q4(x, 1, w, short))  # y too short: rejected before any launch
    eager = dev.gemm_q4(x, 1, w).to_numpy()
    y = dev.alloc(rows)
    g = dev.capture(lambda: dev.gemm_q4(x, 1, w, y))
    try:
        for _ in range(3):
            y.upload(np.zeros(rows, np.float32))
            g.launch()
            dev.sync()
            assert np.array_equal(y.to_numpy(), eager)
    finally:
        g.free()
