"""Dynamic range of the quantized linear paths against the oracle's f64
q4_matvec (crates/tang-infer/src/quantize.rs:256-289), which has no range
limit: activations far above f16's 65504 and far below its 6.1e-5 normal
minimum, reference-quantized weights with f32 block scales below 1e-6, and
rows of very different magnitude in one matrix.  These reach the MFMA GEMM
(m > 16, and m <= 16 when K is too long to stage), the prefill and the MoE
grouped GEMM (T > 64), whose f16 operands are scaled per row by powers of
two.  Tolerances as the other parity tests: max |dev - ref| / max |ref|
below 1e-3 (f32 activations) or 2e-2 (bf16 activations), here also per
output row, so a row of tiny outputs next to large ones is held to its own
scale."""
import numpy as np
import pytest

import oracle
from conftest import max_abs_rel
from moe_ref import CONFIG4, OracleMoe, device_moe, device_moe_forward
from tang_amd import capi

pytestmark = pytest.mark.gpu

TOL_F32, TOL_BF16 = 1e-3, 2e-2


def _per_row_rel(y, ref):
    """Largest max-abs-rel over batch rows, each relative to its own max."""
    return max(max_abs_rel(a, b) for a, b in zip(y, ref))


def _ref(nib, sc, rows, cols, x64):
    return np.stack([oracle.q4_matvec_soa(nib, sc, rows, cols, xr) for xr in x64])


@pytest.mark.parametrize("m", [17, 64, 300])
@pytest.mark.parametrize("mag", [1e5, 3e7, 1e-6, 1e-9])
def test_q4_gemm_bf16_activation_range(dev, m, mag):
    rows, cols = 520, 1000
    print(f"range bf16 m={m} mag={mag}", flush=True)
    nib, sc16 = capi.synth_q4(5, rows, cols)
    sc = oracle.f16_to_f32(sc16)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    xf = capi.synth_normal(6 + m, m * cols, 1.0, capi.F32) * np.float32(mag)
    xb = oracle.f32_to_bf16(xf)
    y = dev.gemm_q4(dev.upload(xb, capi.BF16), m, w).to_numpy().reshape(m, rows)
    ref = _ref(nib, sc, rows, cols, oracle.bf16_to_f32(xb).reshape(m, cols).astype(np.float64))
    err = _per_row_rel(y, ref)
    print("per-row max_abs_rel", err)
    assert np.all(np.isfinite(y))
    assert err < TOL_BF16


@pytest.mark.parametrize("m", [20, 200])
def test_q4_gemm_f32_activations_mixed_rows(dev, m):
    """f32 activations: rows scaled from 1e-8 to 1e8, one row mixing 1e5 and
    1e-5 values, held to the f32 bar."""
    rows, cols = 300, 777
    nib, sc16 = capi.synth_q4(7, rows, cols)
    sc = oracle.f16_to_f32(sc16)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    x = capi.synth_normal(8, m * cols, 1.0, capi.F32).reshape(m, cols)
    x *= np.logspace(-8, 8, m, dtype=np.float64).astype(np.float32)[:, None]
    x[0, ::2] *= np.float32(1e5)
    x[0, 1::2] *= np.float32(1e-5)
    y = dev.gemm_q4(dev.upload(x.reshape(-1)), m, w).to_numpy().reshape(m, rows)
    ref = _ref(nib, sc, rows, cols, x.astype(np.float64))
    err = _per_row_rel(y, ref)
    print("per-row max_abs_rel", err)
    assert err < TOL_F32


@pytest.mark.parametrize("m", [2, 40])
def test_q4_reference_tiny_f32_scales(dev, m):
    """quantize_matrix_q4 on weights of magnitude ~1e-7 (block scales ~1e-7,
    below f16's subnormal range), plus rows of ordinary magnitude in the same
    matrix; f32 activations.  Each output column (weight row) is held to its
    own scale."""
    rows, cols = 96, 640
    rng = np.random.default_rng(12)
    wf = rng.standard_normal((rows, cols)).astype(np.float32)
    wf[: rows // 2] *= np.float32(1e-7)
    wf[rows // 2: rows // 2 + 8] *= np.float32(3e3)
    blocks = oracle.quantize_matrix_q4(wf.reshape(-1), rows, cols)
    assert blocks["scale"][: (rows // 2) * (cols // 32)].max() < 1e-6
    w = dev.q4_upload_blocks(blocks, rows, cols, capi.F32)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    y = dev.gemm_q4(dev.upload(x.reshape(-1)), m, w).to_numpy().reshape(m, rows)
    ref = np.stack([oracle.q4_matvec(blocks, rows, cols, xr.astype(np.float64)) for xr in x])
    err = max(max_abs_rel(y[:, n], ref[:, n]) for n in range(rows))
    print("per-column max_abs_rel", err)
    assert err < TOL_F32


def test_q4_gemm_long_k_small_m(dev):
    """m <= 16 with K too long for the LDS-staged GEMV: the MFMA GEMM with
    one 16-row block, large bf16 activations."""
    rows, cols, m = 64, 40960, 3
    nib, sc16 = capi.synth_q4(9, rows, cols)
    sc = oracle.f16_to_f32(sc16)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    xb = oracle.f32_to_bf16(capi.synth_normal(10, m * cols, 1.0, capi.F32) * np.float32(2e5))
    y = dev.gemm_q4(dev.upload(xb, capi.BF16), m, w).to_numpy().reshape(m, rows)
    ref = _ref(nib, sc, rows, cols, oracle.bf16_to_f32(xb).reshape(m, cols).astype(np.float64))
    err = _per_row_rel(y, ref)
    print("per-row max_abs_rel", err)
    assert err < TOL_BF16


@pytest.mark.parametrize("scale", [1e-3, 300.0])
def test_moe_grouped_gemm_range(dev, scale):
    """Config-4 MoE at T=100 (grouped MFMA GEMM) with the hidden state scaled:
    at 1e-3 the SwiGLU outputs that feed the down projection are ~1e-9 (below
    f16's subnormals), at 300 they exceed 65504.  At 300 the router is nearly
    one-hot and the lower ranks hold probabilities that underflow, so the
    top-1 expert must match exactly and the outputs within the bf16 bar; at
    1e-3 the whole routing must match."""
    cfg, T = CONFIG4, 100
    print(f"moe range scale={scale}", flush=True)
    h = oracle.f32_to_bf16(capi.synth_normal(77, T * cfg["d"], 1.0, capi.F32) * np.float32(scale))
    ref = OracleMoe(cfg, 4)
    r_out, r_idx, r_w = ref.forward(h, T)
    m = device_moe(dev, cfg, 4)
    try:
        out, idx, w = device_moe_forward(dev, m, cfg, h, T)
    finally:
        capi.lib().th_moe_destroy(m)
    if scale < 1:
        assert np.array_equal(idx, r_idx)
    else:
        assert np.array_equal(idx[:, 0], r_idx[:, 0])
    assert np.all(np.isfinite(out))
    err = _per_row_rel(out, r_out)
    print("per-token max_abs_rel", err, "max |out|", float(np.abs(r_out).max()))
    assert err < TOL_BF16
