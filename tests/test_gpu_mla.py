"""MLA absorbed decode (16 heads, qk_nope 128, qk_rope 64,
v_head 128, kv_lora_rank 512, bf16 latent cache) against the oracle's
from-definition or_mla_decode, through the C ABI.  Activations and outputs are
f32, so the bar is 1e-3 max-abs-rel."""
import numpy as np
import pytest

import oracle
from conftest import max_abs_rel
from tang_amd import capi

pytestmark = pytest.mark.gpu

H, DN, DR, R, DV = 16, 128, 64, 512, 128
TOL = 1e-3


def _case(seed, B, L, dn=DN, dr=DR, r=R, dv=DV):
    qn = capi.synth_normal(capi.synth_seed(seed, 0, 0), B * H * dn, 1.0, capi.F32)
    qr = capi.synth_normal(capi.synth_seed(seed, 0, 1), B * H * dr, 1.0, capi.F32)
    cache = capi.synth_normal(capi.synth_seed(seed, 0, 2), B * L * (r + dr), 1.0, capi.BF16)
    wuk, suk = capi.synth_q8_rowwise(capi.synth_seed(seed, 0, 3), H * r, dn)
    wuv, suv = capi.synth_q8_rowwise(capi.synth_seed(seed, 0, 4), H * dv, r)
    return qn, qr, cache, wuk, suk, wuv, suv


def _run(dev, B, L, seed, dn=DN, dr=DR, r=R, dv=DV):
    qn, qr, cache, wuk, suk, wuv, suv = _case(seed, B, L, dn, dr, r, dv)
    scale = 1.0 / np.sqrt(dn + dr)
    ref = oracle.mla_decode(qn, qr, cache, B, H, L, dn, dr, r, dv, wuk, suk, wuv, suv, scale)
    wk = dev.q8_upload_rowwise(wuk, suk, H * r, dn)
    wv = dev.q8_upload_rowwise(wuv, suv, H * dv, r)
    out = dev.mla_decode(dev.upload(qn), dev.upload(qr), dev.upload(cache, capi.BF16), B, H, L, dn, dr, r, dv,
                         wk, wv, scale).to_numpy()
    return out, ref


@pytest.mark.parametrize("B,L", [(8, 4096), (1, 1), (3, 37), (2, 129), (1, 8192), (16, 200)])
def test_mla_matches_oracle(dev, B, L):
    print(f"mla B={B} L={L}", flush=True)
    out, ref = _run(dev, B, L, seed=50 + L)
    err = max_abs_rel(out, ref)
    print("max_abs_rel", err)
    assert np.isfinite(out).all() and err < TOL


def test_mla_small_latent_and_repeat(dev):
    """Other widths (r=64, dr=32, dn=48, dv=32) and two calls in a row sharing
    the device workspace and split counters."""
    for B, L in ((2, 300), (1, 65)):
        out, ref = _run(dev, B, L, seed=7, dn=48, dr=32, r=64, dv=32)
        assert max_abs_rel(out, ref) < TOL


@pytest.mark.parametrize("scale_exp", [18, -18])
def test_mla_cache_far_from_unit_range(dev, scale_exp):
    """A latent cache scaled by 2^18 (o_lat far above f16's 65504) or 2^-18
    (far below f16's normal range): the up-projection's f16 operands are
    scaled by a power of two per head, so the result still matches."""
    B, L = 2, 300
    qn, qr, cache, wuk, suk, wuv, suv = _case(21, B, L)
    c = (cache.astype(np.uint32) << 16).view(np.float32) * np.float32(2.0 ** scale_exp)
    cache = (c.view(np.uint32) >> 16).astype(np.uint16)  # exact: a power-of-two scale of bf16 values
    scale = 1.0 / np.sqrt(DN + DR) * 2.0 ** (-scale_exp)  # scores keep their spread
    ref = oracle.mla_decode(qn, qr, cache, B, H, L, DN, DR, R, DV, wuk, suk, wuv, suv, scale)
    wk = dev.q8_upload_rowwise(wuk, suk, H * R, DN)
    wv = dev.q8_upload_rowwise(wuv, suv, H * DV, R)
    out = dev.mla_decode(dev.upload(qn), dev.upload(qr), dev.upload(cache, capi.BF16), B, H, L, DN, DR, R, DV,
                         wk, wv, scale).to_numpy()
    assert np.isfinite(out).all() and max_abs_rel(out, ref) < TOL


def test_mla_widest_nope_and_rejects_wider(dev):
    """qk_nope 256 (four 64-k chunks of W_UK, the absorb's widest) matches the
    oracle; 260 is rejected with an error, not computed."""
    out, ref = _run(dev, 3, 150, seed=13, dn=256, dr=32, r=64, dv=32)
    assert max_abs_rel(out, ref) < TOL
    qn, qr, cache, wuk, suk, wuv, suv = _case(14, 1, 8, dn=260, dr=32, r=64, dv=32)
    wk = dev.q8_upload_rowwise(wuk, suk, H * 64, 260)
    wv = dev.q8_upload_rowwise(wuv, suv, H * 32, 64)
    with pytest.raises(capi.TangHipError):
        dev.mla_decode(dev.upload(qn), dev.upload(qr), dev.upload(cache, capi.BF16), 1, H, 8, 260, 32, 64, 32, wk, wv,
                       0.1)


def test_mla_graph_replay_matches_eager(dev):
    """th_capture_begin/end around two calls, replayed three times with eager
    calls and synchronisations between the replays: every replay gives the
    eager outputs bit for bit (same kernels, same buffers)."""
    B, L = 2, 700
    qn, qr, cache, wuk, suk, wuv, suv = _case(11, B, L)
    wk = dev.q8_upload_rowwise(wuk, suk, H * R, DN)
    wv = dev.q8_upload_rowwise(wuv, suv, H * DV, R)
    bq, br, bc = dev.upload(qn), dev.upload(qr), dev.upload(cache, capi.BF16)
    bq2 = dev.upload(capi.synth_normal(99, B * H * DN, 1.0, capi.F32))
    scale = 1.0 / np.sqrt(DN + DR)
    out1, out2 = dev.alloc(B * H * DV), dev.alloc(B * H * DV)
    dev.mla_decode(bq, br, bc, B, H, L, DN, DR, R, DV, wk, wv, scale, out1)
    dev.mla_decode(bq2, br, bc, B, H, L, DN, DR, R, DV, wk, wv, scale, out2)
    e1, e2 = out1.to_numpy().copy(), out2.to_numpy().copy()
    g = dev.capture(lambda: (dev.mla_decode(bq, br, bc, B, H, L, DN, DR, R, DV, wk, wv, scale, out1),
                             dev.mla_decode(bq2, br, bc, B, H, L, DN, DR, R, DV, wk, wv, scale, out2)))
    try:
        for rep in range(3):
            out1.upload(np.zeros(B * H * DV, np.float32))
            out2.upload(np.zeros(B * H * DV, np.float32))
            g.launch()
            dev.sync()
            assert np.array_equal(out1.to_numpy(), e1) and np.array_equal(out2.to_numpy(), e2), rep
            dev.mla_decode(bq2, br, bc, B, H, L, DN, DR, R, DV, wk, wv, scale, out1)  # eager work between replays
            dev.sync()
    finally:
        g.free()


def test_mla_rejects_bad_shapes(dev):
    qn, qr, cache, wuk, suk, wuv, suv = _case(1, 1, 8)
    wk = dev.q8_upload_rowwise(wuk, suk, H * R, DN)
    wv = dev.q8_upload_rowwise(wuv, suv, H * DV, R)
    bq, br, bc = dev.upload(qn), dev.upload(qr), dev.upload(cache, capi.BF16)
    with pytest.raises(capi.TangHipError):  # cache buffer too short for L
        dev.mla_decode(bq, br, bc, 1, H, 9, DN, DR, R, DV, wk, wv, 0.1)
    with pytest.raises(capi.TangHipError):  # w_uk / w_uv swapped
        dev.mla_decode(bq, br, bc, 1, H, 8, DN, DR, R, DV, wv, wk, 0.1)
