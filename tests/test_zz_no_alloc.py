"""th_gemm_q4_noalloc, the allocation-free form of th_gemm_q4 (a fixed
per-GPU workspace instead of the device's grow-only allocations): through
the C ABI, against th_gemm_q4 on the same inputs, on two calls in a row
(the second with a smaller input, so it reuses the workspace the first left
behind) and against the oracle's q4_matvec; a size whose prepared
activations exceed the workspace is rejected with an error."""
import ctypes

import numpy as np
import pytest

import oracle
from conftest import max_abs_rel
from tang_amd import capi

pytestmark = pytest.mark.gpu


def _noalloc(dev, x, m, w, rows):
    y = dev.alloc(m * rows)
    capi.check(capi.lib().th_gemm_q4_noalloc(dev.handle, x.handle, m, w.handle, y.handle))
    return y.to_numpy().reshape(m, rows)


def test_noalloc_matches_gemm_q4_on_consecutive_calls(dev):
    rows, cols = 11008, 4096
    nib, sc16 = capi.synth_q4(2, rows, cols)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    for m in (300, 40, 3):  # MFMA with split-K, MFMA with more splits, then the GEMV path
        print(f"noalloc m={m}", flush=True)
        xb = capi.synth_normal(50 + m, m * cols, 1.0, capi.BF16)
        x = dev.upload(xb, capi.BF16)
        got = _noalloc(dev, x, m, w, rows)
        want = dev.gemm_q4(x, m, w).to_numpy().reshape(m, rows)
        assert np.array_equal(got, want), m
        if m == 40:
            ref = np.stack([oracle.q4_matvec_soa(nib, oracle.f16_to_f32(sc16), rows, cols, r)
                            for r in oracle.bf16_to_f32(xb).reshape(m, cols).astype(np.float64)])
            assert max_abs_rel(got, ref) < 2e-2


def test_noalloc_rejects_oversize(dev):
    rows, cols, m = 64, 11008, 4096  # prepared activations: 4096 x 11008 x 2 B > 64 MiB
    nib, sc16 = capi.synth_q4(3, rows, cols)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    x = dev.alloc(m * cols, capi.BF16)
    y = dev.alloc(m * rows)
    rc = capi.lib().th_gemm_q4_noalloc(dev.handle, x.handle, m, w.handle, y.handle)
    assert rc == 1
    assert b"workspace" in capi.lib().th_last_error()
