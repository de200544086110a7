"""Pins the oracle's decode-step composition (or_llama_decode_step,
oracle/tang_oracle.c) against a second, independent restatement: numpy
float64, written here from the reference's decode step
(crates/tang-train/examples/smollm.rs:215-300) and the ComputeDevice ops it
runs through, with the rounding points of the device path spelled out
below.  No oracle function is used to compute the restatement; the oracle is
only run and read.

Rounding points (the ones the decode engine and the oracle both claim):
  * embedding rows and norm weights are bf16 values (exact in f64);
  * every linear's input is rounded to bf16 by bits + 0x7FFF + lsb
    (crates/tang-compute/src/cuda.rs:22-27), weights are (nibble-8)*scale;
  * RoPE tables are computed in f64 and stored f32 (modules.rs:495-511);
  * K rows after RoPE and V rows are stored f16 (the KV cache);
  * everything else (RMSNorm, attention softmax, SwiGLU, residual adds) is
    f64 here and f32 in the oracle, so the two differ by f32 rounding only.

A dropped residual, a swapped norm weight, RoPE on V, a wrong GQA head map,
a missing 1/sqrt(head_dim) or an off-by-one attended range changes the
logits by O(1) relative on checkpoint-scale weights and fails; f32-vs-f64
rounding stays near 4e-8 (bar 1e-6).
"""
import numpy as np
import pytest

from llama_ref import OracleLlama
from tang_amd import capi

T_WQ, T_WK, T_WV, T_WO, T_WG, T_WU, T_WD, T_ATTN_NORM, T_FFN_NORM = range(9)
T_EMBED, T_FINAL_NORM, T_LM_HEAD = 10, 11, 12

TINY = dict(n_layers=2, d_model=64, n_heads=4, n_kv_heads=2, head_dim=16, d_ff=96, vocab=101, max_seq=40, eps=1e-5,
            rope_theta=1e4)
SEED, KV_SEED, PREFILL = 21, 22, 20


def bf16_round(x):
    """f32 -> bf16 by bits + 0x7FFF + lsb (cuda.rs:22-27), returned as f64."""
    b = np.asarray(x, np.float64).astype(np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def bf16_bits_to_f64(h):
    return (np.asarray(h, np.uint32) << 16).view(np.float32).astype(np.float64)


def f16_bits_to_f64(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float64)


def dequant_q4(nib, sc16, rows, cols):
    """Q4Block unpack (quantize.rs:121-132): byte i of a block holds element
    2i in its low nibble and 2i+1 in its high nibble, value = (nibble-8)*scale."""
    bpr = (cols + 31) // 32
    b = nib.reshape(rows, bpr, 16).astype(np.int64)
    q = np.empty((rows, bpr, 32), np.int64)
    q[:, :, 0::2] = b & 15
    q[:, :, 1::2] = b >> 4
    s = f16_bits_to_f64(sc16).reshape(rows, bpr, 1)
    return ((q - 8) * s).reshape(rows, bpr * 32)[:, :cols]


def quantize_q4_np(w):
    """quantize_q4 (quantize.rs:84-118) per row in numpy: scale = amax/7 in
    f32 (1 for an all-zero block), q = round(x * (1/scale)) half away from
    zero, clamped to [-8, 7]; returns (q [rows][cols] int, scales f32
    [rows][blocks])."""
    rows, cols = w.shape
    bpr = (cols + 31) // 32
    wp = np.zeros((rows, bpr * 32), np.float32)
    wp[:, :cols] = w
    blk = wp.reshape(rows, bpr, 32)
    amax = np.max(np.abs(blk), axis=2)
    scale = np.where(amax == 0, np.float32(1), (amax / np.float32(7)).astype(np.float32)).astype(np.float32)
    inv = (np.float32(1) / scale).astype(np.float32)
    v = (blk * inv[:, :, None]).astype(np.float32).astype(np.float64)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -8, 7).astype(np.int64)
    return q.reshape(rows, bpr * 32)[:, :cols], scale


LINEAR = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj", "wo": "self_attn.o_proj",
          "wg": "mlp.gate_proj", "wu": "mlp.up_proj", "wd": "mlp.down_proj"}


def random_tensors(c, seed):
    """Llama tensors (name -> f32) of magnitudes at which every part of the
    step moves the logits: O(1) norm weights and embeddings, linears whose
    outputs are O(1), so attention scores are far from uniform and the MLP
    matters."""
    rng = np.random.default_rng(seed)
    L, d, ff, V, hd = c["n_layers"], c["d_model"], c["d_ff"], c["vocab"], c["head_dim"]
    qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd
    shapes = {"wq": (qd, d), "wk": (kvd, d), "wv": (kvd, d), "wo": (d, qd), "wg": (ff, d), "wu": (ff, d),
              "wd": (d, ff)}
    t = {"model.embed_tokens.weight": rng.normal(0, 1, (V, d)).astype(np.float32),
         "model.norm.weight": rng.normal(1, 0.2, d).astype(np.float32),
         "lm_head.weight": rng.normal(0, 0.3, (V, d)).astype(np.float32)}
    for l in range(L):
        for k, (rows, cols) in shapes.items():
            t["model.layers.%d.%s.weight" % (l, LINEAR[k])] = rng.normal(0, 1.5 / np.sqrt(cols),
                                                                       (rows, cols)).astype(np.float32)
        t["model.layers.%d.input_layernorm.weight" % l] = rng.normal(1, 0.2, d).astype(np.float32)
        t["model.layers.%d.post_attention_layernorm.weight" % l] = rng.normal(1, 0.2, d).astype(np.float32)
    return t


class NumpyLlama:
    """The decode step in numpy float64.  Weights: the seeded synthetic ones
    of th_llama_init_synthetic, or with `tensors` the engine's load of a
    Llama checkpoint (linears through quantize_q4 with f16-rounded block
    scales, embeddings and norm weights rounded to bf16)."""

    def __init__(self, c, seed, kv_seed, prefill, tensors=None):
        self.c = c
        L, d, ff, V = c["n_layers"], c["d_model"], c["d_ff"], c["vocab"]
        hd = c["head_dim"]
        qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd

        def lin(l, tid, rows, cols, name=None):
            if tensors is not None:
                q, sc = quantize_q4_np(tensors[name])
                sc16 = sc.astype(np.float16).astype(np.float64)
                return (q.reshape(rows, -1) * np.repeat(sc16, 32, axis=1)[:, :cols])
            nib, sc = capi.synth_q4(capi.synth_seed(seed, l, tid), rows, cols)
            return dequant_q4(nib, sc, rows, cols)

        def vec(l, tid, n, name=None):
            if tensors is not None:
                return bf16_round(tensors[name].reshape(-1))
            return bf16_bits_to_f64(capi.synth_normal(capi.synth_seed(seed, l, tid), n, 0.02, capi.BF16))

        tids = dict(wq=T_WQ, wk=T_WK, wv=T_WV, wo=T_WO, wg=T_WG, wu=T_WU, wd=T_WD)
        shapes = dict(wq=(qd, d), wk=(kvd, d), wv=(kvd, d), wo=(d, qd), wg=(ff, d), wu=(ff, d), wd=(d, ff))
        self.layers = []
        for l in range(L):
            Wl = {k: lin(l, tids[k], *shapes[k], name="model.layers.%d.%s.weight" % (l, LINEAR[k])) for k in tids}
            Wl["attn_norm"] = vec(l, T_ATTN_NORM, d, "model.layers.%d.input_layernorm.weight" % l)
            Wl["ffn_norm"] = vec(l, T_FFN_NORM, d, "model.layers.%d.post_attention_layernorm.weight" % l)
            self.layers.append(Wl)
        self.embed = vec(L, T_EMBED, V * d, "model.embed_tokens.weight").reshape(V, d)
        self.final_norm = vec(L, T_FINAL_NORM, d, "model.norm.weight")
        self.lm_head = lin(L, T_LM_HEAD, V, d, "lm_head.weight")
        half = hd // 2
        pos = np.arange(c["max_seq"], dtype=np.float64)[:, None]
        freq = 1.0 / np.power(c["rope_theta"], np.arange(half, dtype=np.float64) / half)
        self.cos = np.cos(pos * freq).astype(np.float32).astype(np.float64)
        self.sin = np.sin(pos * freq).astype(np.float32).astype(np.float64)
        # f16 KV cache prefilled with N(0,1) rows (the same generator and seeds)
        self.k = np.zeros((L, c["max_seq"], kvd))
        self.v = np.zeros((L, c["max_seq"], kvd))
        for l in range(L):
            n = prefill * kvd
            self.k[l, :prefill] = f16_bits_to_f64(capi.synth_normal(capi.synth_seed(kv_seed, l, 20), n, 1.0,
                                                                    capi.F16)).reshape(prefill, kvd)
            self.v[l, :prefill] = f16_bits_to_f64(capi.synth_normal(capi.synth_seed(kv_seed, l, 21), n, 1.0,
                                                                    capi.F16)).reshape(prefill, kvd)

    def rms_norm(self, x, w):  # smollm.rs:38-47
        return x * (1.0 / np.sqrt(np.mean(x * x) + self.c["eps"])) * w

    def rope(self, x, n_heads, pos):  # device.rs:582-610, interleaved pairs
        hd = self.c["head_dim"]
        y = x.reshape(n_heads, hd // 2, 2)
        cs, sn = self.cos[pos], self.sin[pos]
        out = np.empty_like(y)
        out[:, :, 0] = y[:, :, 0] * cs - y[:, :, 1] * sn
        out[:, :, 1] = y[:, :, 0] * sn + y[:, :, 1] * cs
        return out.reshape(-1)

    def step(self, token, pos):
        c = self.c
        hd, H, Hkv = c["head_dim"], c["n_heads"], c["n_kv_heads"]
        x = self.embed[token].copy()
        for l, Wl in enumerate(self.layers):
            h = bf16_round(self.rms_norm(x, Wl["attn_norm"]))
            q = self.rope(Wl["wq"] @ h, H, pos)
            k = self.rope(Wl["wk"] @ h, Hkv, pos)
            v = Wl["wv"] @ h
            self.k[l, pos] = k.astype(np.float16).astype(np.float64)
            self.v[l, pos] = v.astype(np.float16).astype(np.float64)
            K, Vv = self.k[l, :pos + 1], self.v[l, :pos + 1]
            att = np.empty(H * hd)
            for hh in range(H):  # smollm.rs:118-176, kv head = h / heads_per_kv
                kv = hh // (H // Hkv)
                s = K[:, kv * hd:(kv + 1) * hd] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                att[hh * hd:(hh + 1) * hd] = p @ Vv[:, kv * hd:(kv + 1) * hd]
            x = x + Wl["wo"] @ bf16_round(att)
            h2 = bf16_round(self.rms_norm(x, Wl["ffn_norm"]))
            g, u = Wl["wg"] @ h2, Wl["wu"] @ h2
            x = x + Wl["wd"] @ bf16_round(g / (1.0 + np.exp(-g)) * u)
        logits = self.lm_head @ bf16_round(self.rms_norm(x, self.final_norm))
        return int(np.argmax(logits)), logits


def _f16_ulps(a_bits, b):
    """|a - b| in units of a's f16 spacing (a given as f16 bit patterns)."""
    a = f16_bits_to_f64(a_bits)
    spacing = np.spacing(np.abs(a).astype(np.float16)).astype(np.float64)
    return np.abs(a - b) / spacing


@pytest.mark.parametrize("weights", ["synthetic", "checkpoint"])
@pytest.mark.parametrize("first_token", [0, 57])
def test_decode_step_composition_matches_numpy_restatement(first_token, weights):
    c = TINY
    tensors = random_tensors(c, 5) if weights == "checkpoint" else None
    ref = OracleLlama(c, SEED, KV_SEED, PREFILL, tensors=tensors)
    npm = NumpyLlama(c, SEED, KV_SEED, PREFILL, tensors=tensors)
    # the inputs agree before any step: same prefilled cache
    assert np.array_equal(f16_bits_to_f64(ref.kc[:, :PREFILL]), npm.k[:, :PREFILL])
    tok_o = tok_n = first_token
    for i in range(6):
        pos = PREFILL + i
        tok_o, lo = ref.step(tok_o, pos)
        tok_n, ln = npm.step(tok_n, pos)
        lo = lo.astype(np.float64)
        err = np.max(np.abs(lo - ln)) / np.max(np.abs(ln))
        gap = np.sort(ln)[-1] - np.sort(ln)[-2]
        print("step %d oracle %d numpy %d rel %.2e gap/max %.2e" % (i, tok_o, tok_n, err, gap / np.abs(ln).max()))
        assert err < 1e-6, (i, err)
        if gap > 1e-3 * np.abs(ln).max():
            assert tok_o == tok_n
        tok_n = tok_o  # follow the oracle's token
        for l in range(c["n_layers"]):  # the appended K/V rows, per layer
            assert np.max(_f16_ulps(ref.kc[l, pos], npm.k[l, pos])) <= 1.0, (i, l)
            assert np.max(_f16_ulps(ref.vc[l, pos], npm.v[l, pos])) <= 1.0, (i, l)
            npm.k[l, pos] = f16_bits_to_f64(ref.kc[l, pos])  # continue from identical caches
            npm.v[l, pos] = f16_bits_to_f64(ref.vc[l, pos])


def test_numpy_quantizer_matches_oracle_blocks():
    """The restatement's own quantize_q4 gives the oracle's blocks."""
    import oracle
    w = np.random.default_rng(3).normal(0, 1, (7, 100)).astype(np.float32)
    w[2, 32:64] = 0.0  # an all-zero block: scale 1
    q, sc = quantize_q4_np(w)
    blocks = oracle.quantize_matrix_q4(w.reshape(-1), 7, 100)
    assert np.array_equal(blocks["scale"].reshape(7, 4), sc)
    nib = blocks["values"].reshape(7, 4, 16).astype(np.int64)
    qo = np.empty((7, 4, 32), np.int64)
    qo[:, :, 0::2] = (nib & 15) - 8
    qo[:, :, 1::2] = (nib >> 4) - 8
    assert np.array_equal(qo.reshape(7, 128)[:, :100], q)


def test_numpy_restatement_sees_plausible_mistakes():
    """The comparison above can fail: on the checkpoint-scale weights each
    plausible composition mistake, made in the restatement, moves the logits
    by far more than the 1e-6 bar."""
    c = TINY
    tensors = random_tensors(c, 5)
    ref = OracleLlama(c, SEED, KV_SEED, PREFILL, tensors=tensors)
    _, lo = ref.step(3, PREFILL)
    lo = lo.astype(np.float64)

    def model():
        return NumpyLlama(c, SEED, KV_SEED, PREFILL, tensors=tensors)

    def rel(m):
        _, lb = m.step(3, PREFILL)
        return np.max(np.abs(lo - lb)) / np.max(np.abs(lb))

    assert rel(model()) < 1e-6
    swapped = model()
    for Wl in swapped.layers:
        Wl["attn_norm"], Wl["ffn_norm"] = Wl["ffn_norm"], Wl["attn_norm"]
    no_rope = model()
    no_rope.rope = lambda x, n, pos: x
    wrong_gqa = model()
    wrong_gqa.layers = [dict(Wl, wk=np.roll(Wl["wk"], c["head_dim"], axis=0),
                             wv=np.roll(Wl["wv"], c["head_dim"], axis=0)) for Wl in wrong_gqa.layers]
    no_mlp = model()
    for Wl in no_mlp.layers:
        Wl["wd"] = np.zeros_like(Wl["wd"])
    no_scale = model()
    no_scale.layers = [dict(Wl, wq=Wl["wq"] * np.sqrt(c["head_dim"])) for Wl in no_scale.layers]
    for name, m in (("swapped norms", swapped), ("no RoPE", no_rope), ("K/V heads swapped", wrong_gqa),
                    ("MLP dropped", no_mlp), ("no 1/sqrt(head_dim)", no_scale)):
        e = rel(m)
        print(name, "%.2e" % e)
        assert e > 1e-2, name
