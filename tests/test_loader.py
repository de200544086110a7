"""Weight loading: the product quantizers
(quantize_matrix_q4/q8, quantize.rs:193-220) against the oracle restatement,
and the safetensors reader against files written by the `safetensors`
package (the format tang-safetensors reads, crates/tang-safetensors/src/lib.rs:11-70).
CPU only; the device upload round trip is in test_gpu_loader.py."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle
from tang_amd import capi


def _cases():
    rng = np.random.default_rng(3)
    yield "normal", rng.normal(0, 1, (37, 200)).astype(np.float32)
    yield "ragged", rng.normal(0, 5, (5, 80)).astype(np.float32)
    z = rng.normal(0, 1, (4, 64)).astype(np.float32)
    z[1] = 0.0  # amax 0: scale 1
    yield "zero-row", z
    # exact halves after scaling: x * (7/amax) lands on .5 -> half away from zero
    h = np.tile(np.array([7.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5] * 4, np.float32), (3, 1))
    yield "halves", h


@pytest.mark.parametrize("name,data", list(_cases()))
def test_quantize_q4_matches_oracle(name, data):
    rows, cols = data.shape
    got = capi.quantize_q4(data, rows, cols)
    want = oracle.quantize_matrix_q4(data, rows, cols)
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("name,data", list(_cases()))
def test_quantize_q8_matches_oracle(name, data):
    rows, cols = data.shape
    got = capi.quantize_q8(data, rows, cols)
    want = oracle.quantize_matrix_q8(data, rows, cols)
    assert got.tobytes() == want.tobytes()


def test_safetensors_read_all_dtypes(tmp_path):
    g = torch.Generator().manual_seed(1)
    ts = {
        "w.f32": torch.randn(7, 9, generator=g, dtype=torch.float32),
        "w.f16": torch.randn(3, 64, generator=g).to(torch.float16),
        "w.bf16": torch.randn(64, 3, generator=g).to(torch.bfloat16),
        "w.f64": torch.randn(11, generator=g, dtype=torch.float64),
        "scalar": torch.tensor(2.5, dtype=torch.float32),
    }
    path = tmp_path / "m.safetensors"
    save_file(ts, str(path), metadata={"format": "pt"})
    f = capi.SafetensorsFile(path)
    info = f.tensors()
    assert info == {"w.f32": ("F32", (7, 9)), "w.f16": ("F16", (3, 64)), "w.bf16": ("BF16", (64, 3)),
                    "w.f64": ("F64", (11,)), "scalar": ("F32", ())}
    for name, t in ts.items():
        want = t.to(torch.float32).reshape(-1).numpy()  # exact except F64, which rounds like a cast
        got = f.read_f32(name, want.size)
        assert got.tobytes() == want.tobytes(), name
    f.close()


def _raw_file(path, header, data=b""):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)


def test_safetensors_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.safetensors"
    _raw_file(p, {"x": {"dtype": "I8", "shape": [2], "data_offsets": [0, 2]}}, b"\0\0")
    with pytest.raises(capi.TangHipError):
        capi.SafetensorsFile(p)  # dtype the reference does not read
    _raw_file(p, {"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8)
    with pytest.raises(capi.TangHipError):
        capi.SafetensorsFile(p)  # offsets disagree with the shape
    p.write_bytes(b"\x05\0\0\0")
    with pytest.raises(capi.TangHipError):
        capi.SafetensorsFile(p)  # truncated length field
    with pytest.raises(capi.TangHipError):
        capi.SafetensorsFile(tmp_path / "missing.safetensors")
