"""C-ABI entry points not exercised through the model paths: buffer
metadata and device-to-device copies (ComputeDevice copy / slice helpers),
quantized-weight metadata, the plain matmul forms of ComputeDevice
(device.rs:103, 407) and the q8 safetensors upload."""
import ctypes

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from tang_amd import capi

pytestmark = pytest.mark.gpu


def test_buffer_info_copy_and_copy_region(dev):
    L = capi.lib()
    src = dev.upload(np.arange(1000, dtype=np.float32))
    dt, n = ctypes.c_int(), ctypes.c_size_t()
    capi.check(L.th_buffer_info(src.handle, ctypes.byref(dt), ctypes.byref(n)))
    assert dt.value == capi.F32 and n.value == 1000
    small = dev.alloc(600)
    small.upload(np.full(600, -1.0, np.float32))
    capi.check(L.th_buffer_copy(small.handle, src.handle))  # min(src, dst) bytes
    assert np.array_equal(small.to_numpy(), np.arange(600, dtype=np.float32))
    dst = dev.alloc(100)
    dst.upload(np.zeros(100, np.float32))
    capi.check(L.th_buffer_copy_region(dst.handle, 50, src.handle, 10, 20))
    want = np.zeros(100, np.float32)
    want[50:70] = np.arange(10, 30, dtype=np.float32)
    assert np.array_equal(dst.to_numpy(), want)
    # out of range: rejected, the destination untouched
    assert L.th_buffer_copy_region(dst.handle, 90, src.handle, 0, 20) != 0
    assert np.array_equal(dst.to_numpy(), want)


def test_qweight_info(dev):
    L = capi.lib()
    nib, sc = capi.synth_q4(1, 100, 256)
    w4 = dev.q4_upload_packed(nib, sc, 100, 256, capi.F16)
    q, rs = capi.synth_q8_rowwise(2, 48, 96)
    w8 = dev.q8_upload_rowwise(q, rs, 48, 96)
    for w, want in ((w4, (100, 256, 4)), (w8, (48, 96, 8))):
        rows, cols, bits = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int()
        capi.check(L.th_qweight_info(w.handle, ctypes.byref(rows), ctypes.byref(cols), ctypes.byref(bits)))
        assert (rows.value, cols.value, bits.value) == want
    w4.free()
    w8.free()


@pytest.mark.parametrize("m,k,n", [(1, 64, 32), (37, 200, 129)])
def test_plain_matmul_forms(dev, m, k, n):
    """th_matmul (A [m][k] x B [k][n]) and th_matmul_b_transposed (B stored
    [n][k]) against float64 numpy; f32 products and accumulation."""
    L = capi.lib()
    rng = np.random.default_rng(m + k + n)
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1, (k, n)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    da, db = dev.upload(a), dev.upload(b)  # held: a temporary's handle would be freed before the call
    c = dev.alloc(m * n)
    capi.check(L.th_matmul(dev.handle, da.handle, db.handle, m, k, n, c.handle))
    got = c.to_numpy().reshape(m, n)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-5
    c2 = dev.alloc(m * n)
    dbt = dev.upload(np.ascontiguousarray(b.T))
    capi.check(L.th_matmul_b_transposed(dev.handle, da.handle, dbt.handle, m, k, n, c2.handle))
    assert np.array_equal(c2.to_numpy(), got.reshape(-1))


def test_safetensors_q8_upload_matches_block_upload(dev, tmp_path):
    """th_st_upload_q8 (quantize_matrix_q8 on upload, quantize.rs:193) gives
    the weight th_q8_upload_blocks makes from the host quantizer's blocks:
    identical GEMV outputs."""
    g = torch.Generator().manual_seed(9)
    w = (torch.randn(64, 160, generator=g) * 0.05).to(torch.float32)
    path = tmp_path / "q8.safetensors"
    save_file({"w": w}, str(path))
    f = capi.SafetensorsFile(path)
    L = capi.lib()
    h = ctypes.c_void_p()
    capi.check(L.th_st_upload_q8(dev.handle, f.handle, b"w", ctypes.byref(h)))
    wst = capi.QWeight(h, 64, 160, 8)
    wblk = dev.q8_upload_blocks(capi.quantize_q8(w.numpy(), 64, 160), 64, 160)
    x = dev.upload(np.random.default_rng(3).normal(0, 1, 160).astype(np.float32))
    y1 = dev.gemv_q8(x, 1, wst).to_numpy()
    y2 = dev.gemv_q8(x, 1, wblk).to_numpy()
    assert np.array_equal(y1, y2)
    wst.free()
    wblk.free()
    f.close()
