"""Pins the CPU oracle (oracle/tang_oracle.c) before it is trusted.

Each check is chosen so a plausible transcription mistake (dropped term,
wrong sign, swapped nibble, transposed index) fails: the reference's own
known-answer tests, exhaustive enumeration where the domain is small,
closed forms, and an independent numpy float64 restatement on small shapes.
"""
import numpy as np
import pytest

import oracle
from conftest import max_abs_rel


# ---------------------------------------------------------------------------
# Reference known-answer tests, crates/tang-infer/src/quantize.rs:297-372
# ---------------------------------------------------------------------------

def test_q8_roundtrip_kat():  # quantize.rs:297-309
    data = np.array([0.5, -1.0, 2.0, -3.0, 0.0, 1.5, -0.7, 0.3], np.float32)
    r = oracle.dequantize_q8(oracle.quantize_q8(data))[: data.size]
    assert np.all(np.abs(data - r) < 0.05)


def test_q4_roundtrip_kat():  # quantize.rs:311-324
    data = np.array([0.5, -1.0, 2.0, -3.0, 0.0, 1.5, -0.7, 0.3], np.float32)
    r = oracle.dequantize_q4(oracle.quantize_q4(data))[: data.size]
    assert np.all(np.abs(data - r) < 1.0)


def test_q8_matvec_basic_kat():  # quantize.rs:326-339
    q = oracle.quantize_matrix_q8(np.array([1, 2, 3, 4, 5, 6], np.float32), 2, 3)
    y = oracle.q8_matvec(q, 2, 3, [1.0, 0.5, -1.0])
    assert abs(y[0] + 1.0) < 0.15 and abs(y[1] - 0.5) < 0.15


def test_q4_matvec_basic_kat():  # quantize.rs:341-353
    q = oracle.quantize_matrix_q4(np.array([1, 2, 3, 4, 5, 6], np.float32), 2, 3)
    y = oracle.q4_matvec(q, 2, 3, [1.0, 0.5, -1.0])
    assert abs(y[0] + 1.0) < 1.5 and abs(y[1] - 0.5) < 1.5
    # Hand-derived exact values: row [1,2,3] -> scale 3/7, q = [2,5,7];
    # row [4,5,6] -> scale 6/7, q = [5,6,7].
    s0, s1 = np.float32(3.0) / np.float32(7.0), np.float32(6.0) / np.float32(7.0)
    e0 = 2 * float(s0) * 1.0 + 5 * float(s0) * 0.5 + 7 * float(s0) * -1.0
    e1 = 5 * float(s1) * 1.0 + 6 * float(s1) * 0.5 + 7 * float(s1) * -1.0
    assert y[0] == pytest.approx(e0, abs=1e-12) and y[1] == pytest.approx(e1, abs=1e-12)


def test_tensor_quantize_roundtrip_kat():  # quantize.rs:355-373
    t = np.array([1.0, -2.0, 3.0, -4.0, 5.0, -6.0], np.float32)
    r = oracle.dequantize_q8(oracle.quantize_q8(t))[:6]
    assert np.all(np.abs(t - r) < 0.1)


# ---------------------------------------------------------------------------
# Bit-level pins of packing and conversions
# ---------------------------------------------------------------------------

def test_q4_unpack_exhaustive():
    """All 256 byte values: low nibble = even element, high = odd, value-8
    (quantize.rs:124-128), scale applied in f32."""
    blocks = np.zeros(16, oracle.Q4_BLOCK)
    allb = np.arange(256, dtype=np.uint8).reshape(16, 16)
    blocks["values"] = allb
    blocks["scale"] = np.float32(0.37)
    out = oracle.dequantize_q4(blocks).reshape(16, 32)
    lo = (allb & 0x0F).astype(np.int32) - 8
    hi = (allb >> 4).astype(np.int32) - 8
    exp = np.empty((16, 32), np.float32)
    exp[:, 0::2] = lo.astype(np.float32) * np.float32(0.37)
    exp[:, 1::2] = hi.astype(np.float32) * np.float32(0.37)
    assert np.array_equal(out, exp)


def test_q4_pack_unpack_identity():
    """quantize(dequantize(b)) == b when the block amax is 7*scale (nibbles in
    1..15, one byte 0xFF): the packing is its own inverse."""
    rng = np.random.default_rng(1)
    for _ in range(64):
        vals = (rng.integers(1, 16, 16, dtype=np.uint8) | (rng.integers(1, 16, 16, dtype=np.uint8) << 4)).astype(np.uint8)
        vals[0] = 0xFF  # element values 7 and 7 -> amax = 7*scale
        blk = np.zeros(1, oracle.Q4_BLOCK)
        blk["values"][0] = vals
        blk["scale"] = np.float32(1.0)
        deq = oracle.dequantize_q4(blk)
        re = oracle.quantize_q4(deq)
        assert np.array_equal(re["values"][0], vals)
        assert re["scale"][0] == np.float32(1.0)


def test_q8_quantize_rounding_half_away():
    # Rust f32::round rounds half away from zero: 2.5 -> 3, -2.5 -> -3.
    data = np.zeros(32, np.float32)
    data[0] = 127.0  # scale 1
    data[1], data[2], data[3] = 2.5, -2.5, 0.49
    b = oracle.quantize_q8(data)
    assert b["scale"][0] == 1.0
    assert list(b["values"][0][:4]) == [127, 3, -3, 0]


def _bf16_ref(x):
    """Independent numpy restatement of bits + 0x7FFF + lsb >> 16."""
    b = x.view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def test_bf16_rne_stratified():
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    for low in (0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1234):
        x = (hi | np.uint32(low)).view(np.float32)
        assert np.array_equal(oracle.f32_to_bf16(x), _bf16_ref(x))
    h = np.arange(1 << 16, dtype=np.uint16)
    assert np.array_equal(oracle.bf16_to_f32(h).view(np.uint32), h.astype(np.uint32) << 16)


def test_f16_conversions_match_numpy():
    h = np.arange(1 << 16, dtype=np.uint16)
    f = oracle.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(f), nan)
    assert np.array_equal(f[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32),
        (rng.standard_normal(100000) * 1e-5).astype(np.float32),   # subnormal range
        (rng.standard_normal(100000) * 3e4).astype(np.float32),    # near overflow
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.0, 2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -25,
                  np.inf, -np.inf], np.float32),
    ])
    assert np.array_equal(oracle.f32_to_f16(x), x.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------
# Matvec: closed forms and an independent numpy restatement
# ---------------------------------------------------------------------------

def _np_dequant_q4(blocks, rows, cols):
    bpr = (cols + 31) // 32
    v = blocks["values"].reshape(rows, bpr, 16)
    q = np.empty((rows, bpr, 32), np.float64)
    q[:, :, 0::2] = (v & 0x0F).astype(np.float64) - 8
    q[:, :, 1::2] = (v >> 4).astype(np.float64) - 8
    s = blocks["scale"].reshape(rows, bpr, 1).astype(np.float64)
    return (q * s).reshape(rows, bpr * 32)[:, :cols]


@pytest.mark.parametrize("rows,cols", [(7, 96), (5, 80), (3, 33), (16, 256)])
def test_q4_matvec_vs_numpy(rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    q = oracle.quantize_matrix_q4(w, rows, cols)
    x = rng.standard_normal(cols)
    y = oracle.q4_matvec(q, rows, cols, x)
    ref = _np_dequant_q4(q, rows, cols) @ x
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("rows,cols", [(7, 96), (5, 80), (4, 31)])
def test_q8_matvec_vs_numpy(rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    q = oracle.quantize_matrix_q8(w, rows, cols)
    bpr = (cols + 31) // 32
    deq = (q["values"].reshape(rows, bpr * 32).astype(np.float64)
           * np.repeat(q["scale"].reshape(rows, bpr).astype(np.float64), 32, axis=1))[:, :cols]
    x = rng.standard_normal(cols)
    assert np.allclose(oracle.q8_matvec(q, rows, cols, x), deq @ x, rtol=1e-12, atol=1e-12)


def test_q4_matvec_integer_closed_form():
    """scale 1 and integer x: the f64 sum is the exact integer dot product."""
    rng = np.random.default_rng(3)
    rows, cols = 9, 320
    bpr = cols // 32
    blocks = np.zeros(rows * bpr, oracle.Q4_BLOCK)
    blocks["values"] = rng.integers(0, 256, (rows * bpr, 16), dtype=np.uint8)
    blocks["scale"] = 1.0
    x = rng.integers(-50, 50, cols).astype(np.float64)
    q = np.empty((rows, cols), np.int64)
    v = blocks["values"].reshape(rows, bpr, 16).astype(np.int64)
    q.reshape(rows, bpr, 32)[:, :, 0::2] = (v & 15) - 8
    q.reshape(rows, bpr, 32)[:, :, 1::2] = (v >> 4) - 8
    exact = q @ x.astype(np.int64)
    assert np.array_equal(oracle.q4_matvec(blocks, rows, cols, x), exact.astype(np.float64))


def test_q4_matvec_one_hot_selects_column():
    rng = np.random.default_rng(4)
    rows, cols = 6, 64
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    q = oracle.quantize_matrix_q4(w, rows, cols)
    deq = _np_dequant_q4(q, rows, cols)  # (nibble-8) * scale, exact in f64
    for c in (0, 1, 31, 32, 63):
        x = np.zeros(cols); x[c] = 1.0
        assert np.array_equal(oracle.q4_matvec(q, rows, cols, x), deq[:, c])


def test_soa_equals_aos_bitwise():
    rng = np.random.default_rng(5)
    rows, cols = 33, 200
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    q = oracle.quantize_matrix_q4(w, rows, cols)
    x = rng.standard_normal(cols)
    a = oracle.q4_matvec(q, rows, cols, x)
    b = oracle.q4_matvec_soa(q["values"].reshape(-1), q["scale"], rows, cols, x, threads=4)
    assert np.array_equal(a, b)
    q8 = oracle.quantize_matrix_q8(w, rows, cols)
    a8 = oracle.q8_matvec(q8, rows, cols, x)
    b8 = oracle.q8_matvec_soa(q8["values"].reshape(-1), q8["scale"], rows, cols, x, threads=3)
    assert np.array_equal(a8, b8)


# ---------------------------------------------------------------------------
# Decode ops: reference KATs (cpu.rs, ops.rs, modules.rs) + numpy restatements
# ---------------------------------------------------------------------------

def test_rms_norm_kat():  # cpu.rs:840-852
    out = oracle.rms_norm(np.array([1, 2, 3, 4], np.float32), np.array([1, 1], np.float32), 2, 2, 1e-5)
    rms0 = np.sqrt(np.float32(2.5) + np.float32(1e-5))
    assert abs(out[0] - 1 / rms0) < 1e-5 and abs(out[1] - 2 / rms0) < 1e-5


def test_rms_norm_vs_numpy():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    out = oracle.rms_norm(x, w, 4, 4096, 1e-5).reshape(4, 4096)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-5) * w
    assert max_abs_rel(out, ref) < 1e-5
    o2, s2 = oracle.rms_norm_residual(x, x[::-1], w, 4, 4096, 1e-5)
    assert np.array_equal(s2.reshape(4, 4096), x + x[::-1])
    assert np.array_equal(o2, oracle.rms_norm(s2, w, 4, 4096, 1e-5))


def test_swiglu_kat():  # ops.rs:216-228
    out = oracle.swiglu(np.array([1.0, -1.0], np.float32), np.array([1.0, 1.0], np.float32))
    assert abs(out[0] - 0.7311) < 1e-3 and abs(out[1] + 0.2689) < 1e-3


def test_rope_identity_at_pos0_and_rotation():  # modules.rs:717, :858
    c, s = oracle.rope_tables(8, 16, 10000.0)
    x = np.arange(16, dtype=np.float32)
    assert np.array_equal(oracle.rope_forward(x, c, s, 1, 2, 8, 0), x)
    y = oracle.rope_forward(x, c, s, 1, 2, 8, 5)
    assert not np.allclose(y, x)
    # pair norms are preserved; numpy restatement of the rotation
    half = 4
    ang = 5 * (1.0 / 10000.0 ** (np.arange(half) / half))
    xr = x.reshape(2, half, 2).astype(np.float64)
    ref = np.stack([xr[..., 0] * np.cos(ang) - xr[..., 1] * np.sin(ang),
                    xr[..., 0] * np.sin(ang) + xr[..., 1] * np.cos(ang)], -1).reshape(-1)
    assert np.allclose(y, ref, atol=1e-5)


def test_kv_attention_kat():  # cpu.rs:938-955
    out = oracle.kv_attention(np.array([1.0, 0.0]), np.array([1.0, 0, 0, 1]), np.array([1.0, 2, 3, 4]), 1, 1, 1, 1, 2)
    s = 1 / np.sqrt(2)
    w0, w1 = np.exp(s) / (np.exp(s) + 1), 1 / (np.exp(s) + 1)
    assert np.allclose(out, [w0 * 1 + w1 * 3, w0 * 2 + w1 * 4], atol=1e-5)


def _np_attention(q, k, v, cache_start, q_len, H, Hkv, D):
    out = np.zeros((q_len, H, D))
    k = k.reshape(-1, Hkv, D).astype(np.float64)
    v = v.reshape(-1, Hkv, D).astype(np.float64)
    q = q.reshape(q_len, H, D).astype(np.float64)
    for i in range(q_len):
        L = cache_start + i + 1
        for h in range(H):
            kh = h // (H // Hkv)
            s = k[:L, kh] @ q[i, h] / np.sqrt(D)
            p = np.exp(s - s.max()); p /= p.sum()
            out[i, h] = p @ v[:L, kh]
    return out.reshape(-1)


def test_kv_attention_vs_numpy_gqa():
    rng = np.random.default_rng(7)
    H, Hkv, D, T, ql = 8, 2, 64, 40, 3
    q = rng.standard_normal(ql * H * D).astype(np.float32)
    k = rng.standard_normal(T * Hkv * D).astype(np.float32)
    v = rng.standard_normal(T * Hkv * D).astype(np.float32)
    out = oracle.kv_attention(q, k, v, 20, ql, H, Hkv, D)
    assert max_abs_rel(out, _np_attention(q, k, v, 20, ql, H, Hkv, D)) < 1e-5


def test_kv_attention_batched_matches_sequential():  # cpu.rs:1095-1135 invariant
    rng = np.random.default_rng(8)
    H, D, T = 4, 16, 12
    q = rng.standard_normal(4 * H * D).astype(np.float32)
    k = rng.standard_normal(T * H * D).astype(np.float32)
    v = rng.standard_normal(T * H * D).astype(np.float32)
    batched = oracle.kv_attention(q, k, v, 5, 4, H, H, D)
    for i in range(4):
        one = oracle.kv_attention(q[i * H * D:(i + 1) * H * D], k, v, 5 + i, 1, H, H, D)
        assert np.array_equal(one, batched[i * H * D:(i + 1) * H * D])


def test_softmax_and_argmax():
    x = np.array([1.0, 3.0, 3.0, -1.0, 2.0, 0.0], np.float32)
    sm = oracle.softmax(x, 2, 3)
    assert abs(sm[:3].sum() - 1) < 1e-6 and abs(sm[3:].sum() - 1) < 1e-6
    assert oracle.argmax(x) == 1  # ties -> lowest index (sampling.rs:184-194)
    assert oracle.argmax(np.full(5, -np.inf, np.float32)) == 0
    assert oracle.argmax(np.array([np.nan, 1.0, np.nan, 2.0], np.float32)) == 3


def test_embedding_kat():  # cpu.rs:1000-1016
    out = oracle.embedding(np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6], np.float32), [2, 0, 1], 3, 2)
    assert np.allclose(out, [0.5, 0.6, 0.1, 0.2, 0.3, 0.4])


# ---- MoE and MLA: no reference implementation; pinned by invariants ----------

def _np_dequant_soa(nib, sc, rows, cols):
    """[rows][cols] f64 from packed nibbles (low nibble = even element) and
    per-group scales: value = (nibble - 8) * scale."""
    b = nib.reshape(rows, -1)
    v = np.empty((rows, b.shape[1] * 2), np.float64)
    v[:, 0::2] = (b & 0x0F).astype(np.int64) - 8
    v[:, 1::2] = (b >> 4).astype(np.int64) - 8
    v = v[:, :cols]
    return v * np.repeat(sc.reshape(rows, -1).astype(np.float64), 32, axis=1)[:, :cols]


def _bf16_round(x):
    return oracle.bf16_to_f32(oracle.f32_to_bf16(np.asarray(x, np.float32))).astype(np.float64)


@pytest.mark.parametrize("topk", [4, 2])
def test_moe_oracle_matches_dense_mixture(topk):
    """out = sum over the top-k experts of p_e * expert_e(h) + shared(h), with p
    the softmax over all router logits (not renormalised) and expert_e computed
    densely from the dequantised weights.  With top-k = E it is the full
    softmax mixture; with top-k < E the chosen set must be the k largest p."""
    from moe_ref import OracleMoe
    from tang_amd import capi
    cfg = dict(d=64, ff=96, E=4, S=1, k=topk)
    om = OracleMoe(cfg, seed=5)
    T = 3
    h = capi.synth_normal(77, T * cfg["d"], 1.0, capi.BF16)
    out, idx, w = om.forward(h, T, threads=1)
    hf = oracle.bf16_to_f32(h).astype(np.float64).reshape(T, cfg["d"])
    router = om.router.astype(np.float64).reshape(cfg["E"], cfg["d"])

    def expert(e, x):
        mats = []
        for tid, rows, cols in ((4, cfg["ff"], cfg["d"]), (5, cfg["ff"], cfg["d"]), (6, cfg["d"], cfg["ff"])):
            nib, sc16 = capi.synth_q4(capi.synth_seed(5, e, tid), rows, cols)
            mats.append(_np_dequant_soa(nib, oracle.f16_to_f32(sc16), rows, cols))
        g = (mats[0] @ x).astype(np.float32).astype(np.float64)
        u = (mats[1] @ x).astype(np.float32).astype(np.float64)
        s = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        return (mats[2] @ _bf16_round(s)).astype(np.float32).astype(np.float64)

    for t in range(T):
        lg = router @ hf[t]
        p = np.exp(lg - lg.max())
        p /= p.sum()
        order = np.argsort(-p, kind="stable")[:topk]
        assert list(idx[t]) == list(order)
        assert np.allclose(w[t], p[order], rtol=1e-5, atol=1e-7)
        ref = sum(p[e] * expert(e, hf[t]) for e in order) + expert(cfg["E"], hf[t])
        assert max_abs_rel(out[t], ref) < 1e-5


def test_mla_oracle_matches_explicit_decompression():
    """Absorbed decode equals attention over the decompressed cache:
    k[t,h] = [W_UK[h]^T c_t ; kr_t], v[t,h] = W_UV[h] c_t, scores
    (q_nope.k_nope + q_rope.kr) * scale, out = sum_t softmax(s) v."""
    rng = np.random.default_rng(11)
    B, H, L, dn, dr, r, dv = 2, 3, 37, 16, 8, 24, 12
    qn = rng.standard_normal(B * H * dn).astype(np.float32)
    qr = rng.standard_normal(B * H * dr).astype(np.float32)
    cache = oracle.f32_to_bf16(rng.standard_normal(B * L * (r + dr)).astype(np.float32))
    wuk = rng.integers(-127, 128, H * r * dn).astype(np.int8)
    wuv = rng.integers(-127, 128, H * dv * r).astype(np.int8)
    suk = rng.uniform(0.005, 0.02, H * r).astype(np.float32)
    suv = rng.uniform(0.005, 0.02, H * dv).astype(np.float32)
    scale = 1.0 / np.sqrt(dn + dr)
    out = oracle.mla_decode(qn, qr, cache, B, H, L, dn, dr, r, dv, wuk, suk, wuv, suv, scale, threads=1)
    c = oracle.bf16_to_f32(cache).astype(np.float64).reshape(B, L, r + dr)
    Wuk = wuk.astype(np.float64).reshape(H, r, dn) * suk.reshape(H, r, 1)
    Wuv = wuv.astype(np.float64).reshape(H, dv, r) * suv.reshape(H, dv, 1)
    ref = np.empty((B, H, dv))
    for b in range(B):
        for h in range(H):
            k_nope = c[b, :, :r] @ Wuk[h]          # [L][dn]: decompressed keys
            v = c[b, :, :r] @ Wuv[h].T              # [L][dv]: decompressed values
            s = (k_nope @ qn.reshape(B, H, dn)[b, h] + c[b, :, r:] @ qr.reshape(B, H, dr)[b, h]) * scale
            pr = np.exp(s - s.max())
            pr /= pr.sum()
            ref[b, h] = pr @ v
    assert max_abs_rel(out, ref.reshape(-1)) < 1e-5


# ---------------------------------------------------------------------------
# Dense operators: matmul, transpose_2d, reduce_sum, bias_add
# (crates/tang-compute/src/cpu.rs:169-199,317-326,760-770; device.rs:378)
# ---------------------------------------------------------------------------

def test_matmul_kats():  # cpu.rs:785-822
    assert oracle.matmul([1, 0, 0, 1], [1, 2, 3, 4], 2, 2, 2).reshape(-1).tolist() == [1, 2, 3, 4]
    assert oracle.matmul([1, 2], [3, 4], 1, 2, 1)[0, 0] == 11.0
    c = oracle.matmul([1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12], 2, 3, 2)
    assert c.reshape(-1).tolist() == [58.0, 64.0, 139.0, 154.0]


def test_matmul_sequential_order_and_numpy():
    """Bit-equal to a sequential f32 loop on a small case (the reference's
    order), and within f32 rounding of numpy float64 on a larger one."""
    rng = np.random.default_rng(4)
    a = rng.standard_normal((3, 7)).astype(np.float32)
    b = rng.standard_normal((7, 5)).astype(np.float32)
    want = np.zeros((3, 5), np.float32)
    for i in range(3):
        for j in range(5):
            s = np.float32(0)
            for p in range(7):
                s = np.float32(s + np.float32(a[i, p] * b[p, j]))
            want[i, j] = s
    assert np.array_equal(oracle.matmul(a, b, 3, 7, 5), want)
    a = rng.standard_normal((40, 300)).astype(np.float32)
    b = rng.standard_normal((300, 33)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert max_abs_rel(oracle.matmul(a, b, 40, 300, 33), ref) < 1e-5
    # a transposed operand would fail this: A is 40x300, A^T B is not defined
    assert not np.allclose(oracle.matmul(a[:33, :33].copy(), b[:33].copy(), 33, 33, 33),
                           (a[:33, :33].T.astype(np.float64) @ b[:33].astype(np.float64)), rtol=1e-3)


def test_transpose_kat_and_numpy():  # cpu.rs:986-994
    assert oracle.transpose_2d([1, 2, 3, 4, 5, 6], 2, 3).tolist() == [1, 4, 2, 5, 3, 6]
    x = np.random.default_rng(1).standard_normal((13, 70)).astype(np.float32)
    assert np.array_equal(oracle.transpose_2d(x, 13, 70), x.T.reshape(-1))


def test_reduce_sum_kats_and_loops():  # cpu.rs:869-890
    d = np.array([1, 2, 3, 4, 5, 6], np.float32)
    assert oracle.reduce_sum(d, [2, 3], 1).tolist() == [6.0, 15.0]
    assert oracle.reduce_sum(d, [2, 3], 0).tolist() == [5.0, 7.0, 9.0]
    rng = np.random.default_rng(2)
    shape = [3, 5, 4]
    x = rng.standard_normal(shape).astype(np.float32)
    for axis in range(3):
        got = oracle.reduce_sum(x.reshape(-1), shape, axis)
        want = np.zeros([s for i, s in enumerate(shape) if i != axis], np.float32)
        moved = np.moveaxis(x, axis, 0)
        for a in range(shape[axis]):  # sequential f32 adds in axis order
            want = (want + moved[a]).astype(np.float32)
        assert np.array_equal(got, want.reshape(-1)), axis


def test_bias_add_vs_numpy():
    rng = np.random.default_rng(3)
    m = rng.standard_normal(6 * 7).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    assert np.array_equal(oracle.bias_add(m, b, 42, 7), (m.reshape(6, 7) + b).reshape(-1))
