"""Safetensors weights into the device layout: a bf16
matrix quantized on upload (quantize_matrix_q4, quantize.rs:208) comes back
bit-exact through th_q4_download_blocks and multiplies like the oracle's
q4_matvec; plain tensors land as f32 / bf16 / f16 device buffers."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle
from conftest import max_abs_rel
from tang_amd import capi

pytestmark = pytest.mark.gpu


def test_safetensors_q4_upload_round_trip_and_gemv(dev, tmp_path):
    print("loader q4 300x520", flush=True)
    g = torch.Generator().manual_seed(5)
    w = (torch.randn(300, 520, generator=g) * 0.05).to(torch.bfloat16)
    path = tmp_path / "w.safetensors"
    save_file({"layer.0.w": w}, str(path))
    f = capi.SafetensorsFile(path)
    qw = f.upload_q4(dev, "layer.0.w")
    w32 = w.to(torch.float32).numpy()
    want = capi.quantize_q4(w32, 300, 520)
    assert qw.download_q4_blocks().tobytes() == want.tobytes()
    x = np.random.default_rng(6).normal(0, 1, 520).astype(np.float32)
    y = dev.gemm_q4(dev.upload(x), 1, qw).to_numpy()
    ref = oracle.q4_matvec(want, 300, 520, x.astype(np.float64))
    assert max_abs_rel(y, ref) < 1e-3
    f.close()


@pytest.mark.parametrize("dtype", [capi.F32, capi.BF16, capi.F16])
def test_safetensors_plain_upload(dev, tmp_path, dtype):
    t = torch.randn(33, 17, generator=torch.Generator().manual_seed(2)).to(torch.float16)
    path = tmp_path / "n.safetensors"
    save_file({"norm": t}, str(path))
    f = capi.SafetensorsFile(path)
    buf = f.upload(dev, "norm", dtype)
    got = buf.to_numpy()
    v = t.to(torch.float32).reshape(-1)
    want = {capi.F32: v.numpy(), capi.BF16: v.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16),
            capi.F16: v.to(torch.float16).view(torch.int16).numpy().view(np.uint16)}[dtype]
    assert got.tobytes() == want.tobytes()
    f.close()
