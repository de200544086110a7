"""MoE layer against the oracle's from-definition MoE.
Routing (top-k indices) must match exactly; the outputs within 2e-2
max-abs-rel (bf16 activations)."""
import numpy as np
import pytest

from conftest import max_abs_rel
from moe_ref import CONFIG4, OracleMoe, device_moe, device_moe_forward
from tang_amd import capi

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [1, 16, 40, 100, 257])  # > 64 tokens: grouped MFMA GEMM
def test_moe_matches_oracle(dev, T):
    cfg = CONFIG4
    print(f"moe T={T}", flush=True)
    h = capi.synth_normal(41 + T, T * cfg["d"], 1.0, capi.BF16)
    ref = OracleMoe(cfg, 4)
    r_out, r_idx, r_w = ref.forward(h, T)
    m = device_moe(dev, cfg, 4)
    try:
        out, idx, w = device_moe_forward(dev, m, cfg, h, T)
    finally:
        capi.lib().th_moe_destroy(m)
    assert np.array_equal(idx, r_idx)
    assert max_abs_rel(w, r_w) < 1e-5
    err = max_abs_rel(out, r_out)
    print("max_abs_rel", err)
    assert err < 2e-2


def test_moe_small_shape_and_repeat(dev):
    """Odd sizes (d=256, ff=96, 8 experts, 1 shared, top-3) and two calls on
    one instance (work buffers reused, counters reset)."""
    cfg = dict(d=256, ff=96, E=8, S=1, k=3)
    ref = OracleMoe(cfg, 9)
    m = device_moe(dev, cfg, 9)
    try:
        for T in (5, 33):
            h = capi.synth_normal(T, T * cfg["d"], 1.0, capi.BF16)
            r_out, r_idx, _ = ref.forward(h, T)
            out, idx, _ = device_moe_forward(dev, m, cfg, h, T)
            assert np.array_equal(idx, r_idx)
            assert max_abs_rel(out, r_out) < 2e-2
    finally:
        capi.lib().th_moe_destroy(m)
