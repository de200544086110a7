"""GPU parity of the decode ops against the CPU oracle (cpu.rs / device.rs
restatements) and the reference's own known-answer tests."""
import numpy as np
import pytest

import oracle
from conftest import max_abs_rel
from tang_amd import capi

pytestmark = pytest.mark.gpu


def test_rms_norm(dev):
    rng = np.random.default_rng(0)
    for groups, dim in [(2, 2), (1, 4096), (3, 1000)]:
        x = rng.standard_normal(groups * dim).astype(np.float32)
        w = rng.standard_normal(dim).astype(np.float32)
        out = dev.rms_norm(dev.upload(x), dev.upload(w), groups, dim, 1e-5).to_numpy()
        assert max_abs_rel(out, oracle.rms_norm(x, w, groups, dim, 1e-5)) < 1e-5
        wb = oracle.f32_to_bf16(w)
        out_b = dev.rms_norm(dev.upload(x), dev.upload(wb, capi.BF16), groups, dim, 1e-5).to_numpy()
        assert max_abs_rel(out_b, oracle.rms_norm(x, oracle.bf16_to_f32(wb), groups, dim, 1e-5)) < 1e-5


def test_rms_norm_residual(dev):
    rng = np.random.default_rng(1)
    a = rng.standard_normal(4096 * 2).astype(np.float32)
    b = rng.standard_normal(4096 * 2).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    o, s = dev.rms_norm_residual(dev.upload(a), dev.upload(b), dev.upload(w), 2, 4096, 1e-5)
    ro, rs = oracle.rms_norm_residual(a, b, w, 2, 4096, 1e-5)
    assert np.array_equal(s.to_numpy(), rs)
    assert max_abs_rel(o.to_numpy(), ro) < 1e-5


def test_rope_bit_exact(dev):
    c, s = capi.rope_tables(128, 2200, 10000.0)
    rng = np.random.default_rng(2)
    x = rng.standard_normal(3 * 32 * 128).astype(np.float32)
    for pos in (0, 5, 2048, 2170):
        out = dev.rope_forward_cached(dev.upload(x[:32 * 128 * 3]), dev.upload(c), dev.upload(s), 3, 32, 128, pos)
        if pos + 3 > 2200:
            continue
        ref = oracle.rope_forward(x, c, s, 3, 32, 128, pos)
        assert np.array_equal(out.to_numpy(), ref), pos


def test_swiglu_add(dev):
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(11008) * 3).astype(np.float32)
    u = rng.standard_normal(11008).astype(np.float32)
    out = dev.swiglu_fused_buf(dev.upload(g), dev.upload(u), 11008).to_numpy()
    ref = oracle.swiglu(g, u)
    assert np.max(np.abs(out.view(np.int32) - ref.view(np.int32))) <= 1  # within 1 ulp of the f64 evaluation
    kat = dev.swiglu_fused_buf(dev.upload([1.0, -1.0]), dev.upload([1.0, 1.0]), 2).to_numpy()
    assert abs(kat[0] - 0.7311) < 1e-3 and abs(kat[1] + 0.2689) < 1e-3  # ops.rs:216-228
    s = dev.add_tensors_buf(dev.upload(g), dev.upload(u), 11008).to_numpy()
    assert np.array_equal(s, oracle.add(g, u))


def test_swiglu_bf16_equals_f64_path_rounded(dev):
    """th_swiglu_bf16 (the f32 evaluation the epilogues use, with the f64
    evaluation near bf16 rounding midpoints) gives exactly the bits of the
    f64 path (th_swiglu) rounded to bf16 by the cuda.rs:22 rule, over 6M
    inputs: N(0, 3) gates, gates over [-120, 120] with up values from 1e-30
    to 1e30 (underflow, overflow of exp), and special values."""
    rng = np.random.default_rng(11)
    n1, n2 = 4 << 20, 2 << 20
    g = np.concatenate([rng.standard_normal(n1) * 3, rng.uniform(-120, 120, n2),
                        [0.0, -0.0, 1e-40, -1e-40, 88.0, -88.0, 104.0, -104.0, np.inf, -np.inf, np.nan, 1.0]])
    u = np.concatenate([rng.standard_normal(n1), rng.choice([-1, 1], n2) * 10.0 ** rng.uniform(-30, 30, n2),
                        [1.0, 1.0, 1.0, -1.0, 1e-30, 1e30, 3.0, -3.0, 1.0, 1.0, 1.0, np.inf]])
    g, u = g.astype(np.float32), u.astype(np.float32)
    n = len(g)
    dg, du = dev.upload(g), dev.upload(u)
    f = dev.swiglu_fused_buf(dg, du, n).to_numpy()
    out = dev.alloc(n, capi.BF16)
    capi.check(capi.lib().th_swiglu_bf16(dev.handle, dg.handle, du.handle, n, out.handle))
    got = out.to_numpy()
    want = oracle.f32_to_bf16(f)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (bad[:5], g[bad[:5]], u[bad[:5]], got[bad[:5]], want[bad[:5]])


def test_embedding(dev):
    w = np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6], np.float32)
    out = dev.embedding(dev.upload(w), dev.upload_u32([2, 0, 1]), 3, 2).to_numpy()
    assert np.array_equal(out, oracle.embedding(w, [2, 0, 1], 3, 2))  # cpu.rs:1000-1016
    with pytest.raises(capi.TangHipError):
        dev.embedding(dev.upload(w), dev.upload_u32([3]), 1, 2)
    wb = capi.synth_normal(4, 32000 * 64, 0.02, capi.BF16)
    ids = [1, 31999, 17]
    out = dev.embedding(dev.upload(wb, capi.BF16), dev.upload_u32(ids), 3, 64).to_numpy()
    assert np.array_equal(out, oracle.embedding(oracle.bf16_to_f32(wb), ids, 3, 64))


def test_softmax_argmax(dev):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(3 * 32000).astype(np.float32)
    sm = dev.softmax(dev.upload(x), 3, 32000).to_numpy()
    assert max_abs_rel(sm, oracle.softmax(x, 3, 32000)) < 1e-5
    am = dev.argmax(dev.upload(x), 3, 32000).to_numpy()
    assert list(am) == [oracle.argmax(x[i * 32000:(i + 1) * 32000]) for i in range(3)]
    ties = np.array([1.0, 5.0, 2.0, 5.0, 5.0] + [0.0] * 1000, np.float32)
    assert dev.argmax(dev.upload(ties), 1, ties.size).to_numpy()[0] == 1
    allinf = np.full(300, -np.inf, np.float32)
    assert dev.argmax(dev.upload(allinf), 1, 300).to_numpy()[0] == 0


def test_kv_attention_kat(dev):  # cpu.rs:938-955
    out = dev.kv_attention(dev.upload([1.0, 0.0]), dev.upload([1.0, 0, 0, 1]), dev.upload([1.0, 2, 3, 4]),
                           1, 1, 1, 1, 2).to_numpy()
    ref = oracle.kv_attention(np.array([1.0, 0.0]), np.array([1.0, 0, 0, 1]), np.array([1.0, 2, 3, 4]), 1, 1, 1, 1, 2)
    assert max_abs_rel(out, ref) < 1e-6


@pytest.mark.parametrize("H,Hkv,D,start,ql,f16", [
    (32, 32, 128, 2048, 1, True),     # config-3 decode step
    (32, 32, 128, 2175, 1, True),     # past the reference CUDA kernel's 2048 cap
    (8, 2, 64, 100, 4, False),        # GQA, batched causal queries
    (4, 4, 256, 700, 2, True),
    (6, 3, 20, 33, 3, False),         # untuned head_dim -> generic kernel
])
def test_kv_attention(dev, H, Hkv, D, start, ql, f16):
    print(f"attention H={H} Hkv={Hkv} D={D} start={start} ql={ql} f16={f16}", flush=True)
    rng = np.random.default_rng(H + D + start)
    T = start + ql
    q = rng.standard_normal(ql * H * D).astype(np.float32)
    k = rng.standard_normal(T * Hkv * D).astype(np.float32)
    v = rng.standard_normal(T * Hkv * D).astype(np.float32)
    if f16:
        kh, vh = oracle.f32_to_f16(k), oracle.f32_to_f16(v)
        kb, vb = dev.upload(kh, capi.F16), dev.upload(vh, capi.F16)
        k, v = oracle.f16_to_f32(kh), oracle.f16_to_f32(vh)
    else:
        kb, vb = dev.upload(k), dev.upload(v)
    out = dev.kv_attention(dev.upload(q), kb, vb, start, ql, H, Hkv, D).to_numpy()
    ref = oracle.kv_attention(q, k, v, start, ql, H, Hkv, D)
    err = max_abs_rel(out, ref)
    print("max_abs_rel", err)
    assert err < 1e-4


def test_convert_roundtrip(dev):
    x = np.concatenate([capi.synth_normal(1, 5000), np.array([65504.0, 1e-7, -0.0], np.float32)]).astype(np.float32)
    b = dev.convert(dev.upload(x), capi.BF16).to_numpy()
    assert np.array_equal(b, oracle.f32_to_bf16(x))
    h = dev.convert(dev.upload(x), capi.F16).to_numpy()
    assert np.array_equal(h, oracle.f32_to_f16(x))
    back = dev.convert(dev.upload(h, capi.F16), capi.F32).to_numpy()
    assert np.array_equal(back, oracle.f16_to_f32(h))
    z = dev.upload(x)
    dev.zero_buffer(z)
    assert not z.to_numpy().any()


def test_objects_freed_after_device_close():
    # Buffers and weights may be freed (explicitly or by the garbage
    # collector) after their device was destroyed; the free must not read
    # the destroyed device.
    d = capi.HipComputeDevice(0)
    rows, cols = 64, 256
    nib, sc16 = capi.synth_q4(2, rows, cols)
    w = d.q4_upload_packed(nib, sc16, rows, cols, capi.F16)
    x = d.upload(capi.synth_normal(3, cols, 1.0, capi.BF16), capi.BF16)
    y = d.gemm_q4(x, 1, w)
    ref = oracle.q4_matvec_soa(nib, oracle.f16_to_f32(sc16), rows, cols,
                               oracle.bf16_to_f32(capi.synth_normal(3, cols, 1.0, capi.BF16)).astype(np.float64))
    assert max_abs_rel(y.to_numpy(), ref) < 2e-2
    d.close()
    w.free()
    x.free()
    del y  # freed by its finaliser, also after the device
