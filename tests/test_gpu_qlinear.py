"""GPU parity of the quantized linear kernels against the CPU oracle
(q4_matvec / q8_matvec of crates/tang-infer/src/quantize.rs:227-289).

Tolerances (max |dev - ref| / max |ref|): 1e-3 with f32 activations,
2e-2 with bf16 activations.  Weight packing is checked bit-exactly.
"""
import numpy as np
import pytest

import oracle
from conftest import max_abs_rel
from tang_amd import capi

pytestmark = pytest.mark.gpu

TOL_F32, TOL_BF16 = 1e-3, 2e-2


def _q4_case(rows, cols, seed):
    nib, sc16 = capi.synth_q4(seed, rows, cols)
    sc = oracle.f16_to_f32(sc16)
    return nib, sc16, sc


def _ref_q4(nib, sc, rows, cols, x_f64):
    return np.stack([oracle.q4_matvec_soa(nib, sc, rows, cols, xr) for xr in x_f64])


@pytest.mark.parametrize("rows,cols", [(11008, 4096), (4096, 11008), (16, 128), (37, 200), (5, 3)])
@pytest.mark.parametrize("m", [1, 2, 4, 6, 8, 11, 16])  # 5..16 rows: 8/16-row blocks with live-row masking
def test_q4_gemv_bf16_activations(dev, rows, cols, m):
    print(f"q4 gemv bf16 rows={rows} cols={cols} m={m}", flush=True)
    nib, sc16, sc = _q4_case(rows, cols, 11 + rows + m)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    xb = capi.synth_normal(99 + m, m * cols, 1.0, capi.BF16)
    x = dev.upload(xb, capi.BF16)
    y = dev.gemm_q4(x, m, w).to_numpy().reshape(m, rows)
    ref = _ref_q4(nib, sc, rows, cols, oracle.bf16_to_f32(xb).reshape(m, cols).astype(np.float64))
    err = max_abs_rel(y, ref)
    print("max_abs_rel", err)
    assert err < TOL_BF16


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (300, 520)])
@pytest.mark.parametrize("m", [1, 3, 6, 8])
def test_q4_gemv_f32_activations(dev, rows, cols, m):
    print(f"q4 gemv f32 rows={rows} cols={cols} m={m}", flush=True)
    nib, sc16, sc = _q4_case(rows, cols, 5 + m)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    xf = capi.synth_normal(7 + m, m * cols, 1.0, capi.F32)
    y = dev.gemm_q4(dev.upload(xf), m, w).to_numpy().reshape(m, rows)
    ref = _ref_q4(nib, sc, rows, cols, xf.reshape(m, cols).astype(np.float64))
    err = max_abs_rel(y, ref)
    print("max_abs_rel", err)
    assert err < TOL_F32


@pytest.mark.parametrize("m", [9, 16, 40, 64, 130, 1100])  # 1100: the 128-row column blocks
def test_q4_gemm_mfma(dev, m):
    rows, cols = 1000, 1536
    print(f"q4 mfma m={m}", flush=True)
    nib, sc16, sc = _q4_case(rows, cols, 31 + m)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    xb = capi.synth_normal(3 + m, m * cols, 1.0, capi.BF16)
    y = dev.gemm_q4(dev.upload(xb, capi.BF16), m, w).to_numpy().reshape(m, rows)
    ref = _ref_q4(nib, sc, rows, cols, oracle.bf16_to_f32(xb).reshape(m, cols).astype(np.float64))
    err = max_abs_rel(y, ref)
    print("max_abs_rel", err)
    assert err < TOL_BF16


def test_q4_gemm_mfma_f32_activations(dev):
    """The GEMM's one-pass activation conversion from f32 (ragged K)."""
    rows, cols, m = 300, 1000, 70
    nib, sc16, sc = _q4_case(rows, cols, 8)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    xf = capi.synth_normal(9, m * cols, 1.0, capi.F32)
    y = dev.gemm_q4(dev.upload(xf), m, w).to_numpy().reshape(m, rows)
    ref = _ref_q4(nib, sc, rows, cols, xf.reshape(m, cols).astype(np.float64))
    err = max_abs_rel(y, ref)
    print("max_abs_rel", err)
    assert err < TOL_F32


@pytest.mark.parametrize("rows,cols,m", [(11008, 4096, 8), (11008, 4096, 16), (11008, 4096, 13),
                                         (4096, 11008, 7), (4096, 11008, 12)])
def test_q4_config2_batched(dev, rows, cols, m):
    """Multi-tile workgroups over the config-2 shape; K=11008 with 8+ rows
    overflows the LDS staging and takes the MFMA GEMM instead."""
    nib, sc16, sc = _q4_case(rows, cols, 2)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    xb = capi.synth_normal(20 + m, m * cols, 1.0, capi.BF16)
    y = dev.gemm_q4(dev.upload(xb, capi.BF16), m, w).to_numpy().reshape(m, rows)
    ref = _ref_q4(nib, sc, rows, cols, oracle.bf16_to_f32(xb).reshape(m, cols).astype(np.float64))
    err = max_abs_rel(y, ref)
    print(f"q4 config2 m={m} max_abs_rel {err}")
    assert err < TOL_BF16


@pytest.mark.parametrize("rows", [9600, 6000])  # 600 / 375 tiles: three / two per workgroup, side by side
@pytest.mark.parametrize("cols", [130, 256, 1000])  # one to eight 128-wide items: a wave may hold one item
@pytest.mark.parametrize("m,dt", [(3, "bf16"), (4, "bf16"), (8, "bf16"), (16, "bf16"), (2, "f32"), (4, "f32"),
                                  (7, "f32")])
def test_q4_gemv_side_by_side_tiles_short_k(dev, rows, cols, m, dt):
    """Workgroups streaming two or three tiles side by side, on short K,
    where a wave's staging region is smaller than its partials of all the
    tiles (the region is sized for both)."""
    print(f"q4 side-by-side rows={rows} cols={cols} m={m} {dt}", flush=True)
    nib, sc16, sc = _q4_case(rows, cols, 31 + m)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    if dt == "bf16":
        xb = capi.synth_normal(40 + m, m * cols, 1.0, capi.BF16)
        y = dev.gemm_q4(dev.upload(xb, capi.BF16), m, w).to_numpy().reshape(m, rows)
        ref = _ref_q4(nib, sc, rows, cols, oracle.bf16_to_f32(xb).reshape(m, cols).astype(np.float64))
        tol = TOL_BF16
    else:
        xf = capi.synth_normal(40 + m, m * cols, 1.0, capi.F32)
        y = dev.gemm_q4(dev.upload(xf), m, w).to_numpy().reshape(m, rows)
        ref = _ref_q4(nib, sc, rows, cols, xf.reshape(m, cols).astype(np.float64))
        tol = TOL_F32
    err = max_abs_rel(y, ref)
    print("max_abs_rel", err)
    assert err < tol


def test_q4_reference_blocks_f32_scales(dev):
    """Weights produced by the reference quantizer (f32 scales, ragged K)."""
    rng = np.random.default_rng(0)
    rows, cols = 70, 301
    wf = rng.standard_normal((rows, cols)).astype(np.float32)
    blocks = oracle.quantize_matrix_q4(wf, rows, cols)
    w = dev.q4_upload_blocks(blocks, rows, cols, capi.F32)
    back = w.download_q4_blocks()
    assert np.array_equal(back.view(np.uint8), blocks.view(np.uint8))  # bit-exact round trip
    x = rng.standard_normal((2, cols)).astype(np.float32)
    y = dev.gemm_q4(dev.upload(x), 2, w).to_numpy().reshape(2, rows)
    ref = np.stack([oracle.q4_matvec(blocks, rows, cols, xr.astype(np.float64)) for xr in x])
    assert max_abs_rel(y, ref) < TOL_F32


def test_q4_integer_closed_form_exact(dev):
    """Scale 1, integer activations: the f32 device sum is exact (|sum| < 2^24)."""
    rows, cols = 64, 1024
    nib, _ = capi.synth_q4(77, rows, cols)
    ones = np.full((rows, cols // 32), 0x3C00, np.uint16)  # f16 1.0
    w = dev.q4_upload_packed(nib, ones, rows, cols, capi.F16)
    rng = np.random.default_rng(1)
    x = rng.integers(-20, 21, cols).astype(np.float32)
    y = dev.gemm_q4(dev.upload(x), 1, w).to_numpy()
    ref = oracle.q4_matvec_soa(nib, np.ones((rows, cols // 32), np.float32), rows, cols, x.astype(np.float64))
    assert np.array_equal(y.astype(np.float64), ref)


def test_q4_one_hot_selects_column_exact(dev):
    rows, cols = 48, 256
    nib, sc16, sc = _q4_case(rows, cols, 4)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    for c in (0, 7, 8, 31, 32, 200, 255):
        x = np.zeros(cols, np.float32); x[c] = 1.0
        y = dev.gemm_q4(dev.upload(x), 1, w).to_numpy()
        ref = oracle.q4_matvec_soa(nib, sc, rows, cols, x.astype(np.float64))
        assert np.array_equal(y.astype(np.float64), ref.astype(np.float32).astype(np.float64)), c


def test_q4_f16_scale_upload_rejects_inexact(dev):
    blocks = np.zeros(1, capi.Q4_BLOCK)
    blocks["scale"] = np.float32(0.1)  # not an f16 value
    with pytest.raises(capi.TangHipError):
        dev.q4_upload_blocks(blocks, 1, 32, capi.F16)


@pytest.mark.parametrize("rows,cols,m", [(4096, 4096, 1), (1000, 700, 3), (7, 3, 2), (512, 128, 6)])
def test_q8_gemv_rowwise(dev, rows, cols, m):
    print(f"q8 rows={rows} cols={cols} m={m}", flush=True)
    q, rs = capi.synth_q8_rowwise(1, rows, cols)
    w = dev.q8_upload_rowwise(q, rs, rows, cols)
    x = capi.synth_normal(2, m * cols, 1.0, capi.F32)
    y = dev.gemv_q8(dev.upload(x), m, w).to_numpy().reshape(m, rows)
    bpr = (cols + 31) // 32
    qp = np.zeros((rows, bpr * 32), np.int8); qp[:, :cols] = q
    scales = np.repeat(rs[:, None], bpr, axis=1)
    ref = np.stack([oracle.q8_matvec_soa(qp, scales, rows, cols, xr.astype(np.float64))
                    for xr in x.reshape(m, cols)])
    err = max_abs_rel(y, ref)
    print("max_abs_rel", err)
    assert err < TOL_F32


def test_q8_reference_blocks_per_group_scales(dev):
    rng = np.random.default_rng(3)
    rows, cols = 50, 200
    wf = rng.standard_normal((rows, cols)).astype(np.float32)
    blocks = oracle.quantize_matrix_q8(wf, rows, cols)
    w = dev.q8_upload_blocks(blocks, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    y = dev.gemv_q8(dev.upload(x), 1, w).to_numpy()
    ref = oracle.q8_matvec(blocks, rows, cols, x.astype(np.float64))
    assert max_abs_rel(y, ref) < TOL_F32


def test_reference_kats_on_device(dev):
    """q8_matvec_basic / q4_matvec_basic (quantize.rs:326-353) through the device."""
    wf = np.array([1, 2, 3, 4, 5, 6], np.float32)
    x = dev.upload(np.array([1.0, 0.5, -1.0], np.float32))
    q8 = oracle.quantize_matrix_q8(wf, 2, 3)
    y8 = dev.gemv_q8(x, 1, dev.q8_upload_blocks(q8, 2, 3)).to_numpy()
    assert abs(y8[0] + 1.0) < 0.15 and abs(y8[1] - 0.5) < 0.15
    q4 = oracle.quantize_matrix_q4(wf, 2, 3)
    y4 = dev.gemm_q4(x, 1, dev.q4_upload_blocks(q4, 2, 3, capi.F32)).to_numpy()
    ref4 = oracle.q4_matvec(q4, 2, 3, [1.0, 0.5, -1.0])
    assert np.allclose(y4, ref4, rtol=1e-6, atol=1e-6)


def test_full_size_linearity(dev):
    """Size-independent property at config-2 shape: W(a x1 + x2) = a W x1 + W x2."""
    rows, cols = 11008, 4096
    nib, sc16, _ = _q4_case(rows, cols, 2)
    w = dev.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    x1 = capi.synth_normal(1, cols); x2 = capi.synth_normal(2, cols)
    y1 = dev.gemm_q4(dev.upload(x1), 1, w).to_numpy()
    y2 = dev.gemm_q4(dev.upload(x2), 1, w).to_numpy()
    y3 = dev.gemm_q4(dev.upload(2.0 * x1 + x2), 1, w).to_numpy()
    assert max_abs_rel(y3, 2.0 * y1 + y2) < 1e-4
