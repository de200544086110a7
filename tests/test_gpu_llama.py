"""Decode-engine parity: greedy tokens identical to the CPU oracle's.

Small config: compared live with the oracle (GQA, head_dim 64).
7B config: 128 greedy steps from position 2048 compared
with tests/golden/llama7b_decode.json, which tests/golden/make_decode_golden.py
wrote by running the oracle on the same seeded synthetic model.
"""
import ctypes
import json
import os

import numpy as np
import pytest

import oracle
from conftest import max_abs_rel
from llama_ref import CONFIG_7B, CONFIG_SMALL, OracleLlama, device_generate, device_llama
from tang_amd import capi

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "llama7b_decode.json")


def test_small_llama_matches_oracle(dev):
    cfg = CONFIG_SMALL
    seed, kv_seed, prefill, steps = 7, 8, 100, 48
    ref = OracleLlama(cfg, seed, kv_seed, prefill)
    r_toks, margins, r_logits = ref.generate(1, prefill, steps)
    m = device_llama(dev, cfg, seed, kv_seed, prefill)
    try:
        toks, logits = device_generate(m, cfg, 1, prefill, steps)
    finally:
        capi.lib().th_llama_destroy(m)
    print("oracle", r_toks[:16], "min margin %.3e" % min(margins))
    print("device", list(toks[:16]))
    assert list(toks) == r_toks
    assert max_abs_rel(logits, r_logits) < 1e-3


def test_narrow_model_wide_ffn_matches_oracle(dev):
    """d_model 256 with an 11008-wide FFN and a 22016-row LM head: the
    gate/up and LM-head GEMVs take two tiles per workgroup side by side on
    a K short enough that a wave holds a single 128-wide item."""
    cfg = dict(CONFIG_SMALL, n_layers=1, d_ff=11008, vocab=22016)
    seed, kv_seed, prefill, steps = 5, 6, 40, 12
    ref = OracleLlama(cfg, seed, kv_seed, prefill)
    r_toks, margins, r_logits = ref.generate(1, prefill, steps)
    m = device_llama(dev, cfg, seed, kv_seed, prefill)
    try:
        toks, logits = device_generate(m, cfg, 1, prefill, steps)
    finally:
        capi.lib().th_llama_destroy(m)
    print("oracle", r_toks, "min margin %.3e" % min(margins))
    print("device", list(toks))
    assert list(toks) == r_toks
    assert max_abs_rel(logits, r_logits) < 1e-3


def test_small_llama_long_context_matches_oracle(dev):
    """Positions past 4096: more than sixteen 256-position attention splits,
    so the last split's merge takes a second round of records."""
    cfg = dict(CONFIG_SMALL, max_seq=4608)
    seed, kv_seed, prefill, steps = 7, 8, 4400, 8
    ref = OracleLlama(cfg, seed, kv_seed, prefill)
    r_toks, margins, r_logits = ref.generate(1, prefill, steps)
    m = device_llama(dev, cfg, seed, kv_seed, prefill)
    try:
        toks, logits = device_generate(m, cfg, 1, prefill, steps)
    finally:
        capi.lib().th_llama_destroy(m)
    print("oracle", r_toks, "min margin %.3e" % min(margins))
    print("device", list(toks))
    assert list(toks) == r_toks
    assert max_abs_rel(logits, r_logits) < 1e-3


def test_small_llama_generation_is_resumable(dev):
    """Two generate calls (24 + 24 steps) equal one 48-step call: the KV cache
    and position live on the device (kv_cache.rs:76-100 append semantics)."""
    cfg = CONFIG_SMALL
    m = device_llama(dev, cfg, 7, 8, 100)
    try:
        full, _ = device_generate(m, cfg, 1, 100, 48)
        capi.check(capi.lib().th_llama_fill_kv_synthetic(m, 100, 8))
        a, _ = device_generate(m, cfg, 1, 100, 24)
        b, _ = device_generate(m, cfg, int(a[-1]), 124, 24)
    finally:
        capi.lib().th_llama_destroy(m)
    assert list(full) == list(a) + list(b)


def test_llama_rejects_overrun(dev):
    cfg = CONFIG_SMALL
    m = device_llama(dev, cfg, 7, 8, 100)
    try:
        with pytest.raises(capi.TangHipError):
            device_generate(m, cfg, 1, cfg["max_seq"] - 2, 4)
        with pytest.raises(capi.TangHipError):
            device_generate(m, cfg, cfg["vocab"], 100, 1)
    finally:
        capi.lib().th_llama_destroy(m)


# A decision is numerically determined when the oracle's top-2 logit gap
# exceeds this fraction of the step's largest |logit|: closer calls depend on
# summation order, in the oracle too.
DECIDED = 1e-3
# Per-step logit bar of the teacher-forced check, as a fraction of the step's
# largest |logit|.  Linear inputs are bf16 (north-star bar 2e-2); the device's
# own f16 K/V rows of the new positions add ~1e-3 by step 100, so the bar is
# 2e-3, and a token within it of the oracle's maximum counts as a tie.
LOGIT_TOL = 2e-3


def _golden():
    return json.load(open(GOLDEN))


@pytest.mark.skipif(not os.path.exists(GOLDEN), reason="golden vectors not generated")
def test_7b_decode_free_running_matches_golden(dev):
    """128 greedy steps from position 2048: all 128 tokens identical to the
    oracle's, and the final logits within the bf16-activation bar."""
    g = _golden()
    cfg = CONFIG_7B
    m = device_llama(dev, cfg, g["seed"], g["kv_seed"], g["prefill"])
    try:
        toks, logits = device_generate(m, cfg, g["first_token"], g["prefill"], g["steps"])
    finally:
        capi.lib().th_llama_destroy(m)
    mism = [i for i, (a, b) in enumerate(zip(toks, g["tokens"])) if a != b]
    print("min margin %.3e; mismatching steps %s" % (min(g["margins"]), mism[:8]))
    assert list(toks) == g["tokens"]
    # after 128 autoregressive steps the device's own KV rows feed every step:
    # differences compound, so the bar is the bf16-activation one (linear
    # inputs are bf16 as in cuda.rs:22); single steps are held to LOGIT_TOL
    # by the teacher-forced tests
    last = np.array(g["last_logits_head"], np.float32)
    assert max_abs_rel(logits[: last.size], last) < 2e-2


@pytest.mark.skipif(not os.path.exists(GOLDEN), reason="golden vectors not generated")
def test_7b_decode_teacher_forced_128_steps(dev):
    """Every one of the 128 steps, fed the oracle's previous token: the
    device's logits at the oracle's five largest agree to LOGIT_TOL of the
    step's largest |logit|, and its token is the oracle's or one within that
    bar of the oracle's maximum."""
    g = _golden()
    cfg = CONFIG_7B
    m = device_llama(dev, cfg, g["seed"], g["kv_seed"], g["prefill"])
    exact = 0
    try:
        for i in range(g["steps"]):
            tok_in = g["first_token"] if i == 0 else g["tokens"][i - 1]
            toks, logits = device_generate(m, cfg, tok_in, g["prefill"] + i, 1)
            ids, vals, amax = g["top5_ids"][i], g["top5_logits"][i], g["logit_absmax"][i]
            tol = LOGIT_TOL * amax
            dev_vals = logits[ids]
            assert np.max(np.abs(dev_vals - np.array(vals, np.float32))) <= tol, (i, dev_vals, vals)
            tied = [j for j, v in zip(ids, vals) if v >= vals[0] - tol]
            assert int(toks[0]) in tied, (i, int(toks[0]), ids, vals)
            exact += int(toks[0]) == g["tokens"][i]
    finally:
        capi.lib().th_llama_destroy(m)
    print("steps with the oracle's exact token: %d / %d" % (exact, g["steps"]))


FORCED = os.path.join(os.path.dirname(__file__), "golden", "llama7b_forced.json")


@pytest.mark.skipif(not os.path.exists(FORCED), reason="golden vectors not generated")
def test_7b_decode_teacher_forced_distinct_tokens(dev):
    """128 steps on 128 distinct seeded input tokens (each step reads a
    different embedding row and appends its own K/V rows): the first 256
    logits and the oracle's five largest agree to LOGIT_TOL of the step's
    largest |logit|, and the token equals the oracle's wherever the oracle's
    top-2 gap decides it (otherwise it is one tied within the bar)."""
    g = json.load(open(FORCED))
    cfg = CONFIG_7B
    m = device_llama(dev, cfg, g["seed"], g["kv_seed"], g["prefill"])
    exact = decided = 0
    try:
        for i, tok_in in enumerate(g["tokens_in"]):
            toks, logits = device_generate(m, cfg, tok_in, g["prefill"] + i, 1)
            amax = g["logit_absmax"][i]
            tol = LOGIT_TOL * amax
            head = np.array(g["logits_head"][i], np.float32)
            assert np.max(np.abs(logits[: head.size] - head)) <= tol, i
            ids, vals = g["top5_ids"][i], g["top5_logits"][i]
            assert np.max(np.abs(logits[ids] - np.array(vals, np.float32))) <= tol, i
            if g["margins"][i] > DECIDED * amax:
                decided += 1
                assert int(toks[0]) == g["tokens"][i], (i, int(toks[0]), g["tokens"][i])
            else:
                assert int(toks[0]) in [j for j, v in zip(ids, vals) if v >= vals[0] - tol], i
            exact += int(toks[0]) == g["tokens"][i]
    finally:
        capi.lib().th_llama_destroy(m)
    print("exact tokens %d / %d (%d decided by the oracle)" % (exact, len(g["tokens_in"]), decided))


def _device_steps_oracle_sampler(dev, cfg, prompt, prefill, steps, seed, stop=None, **kw):
    """generate() (sampling.rs:229-256) composed in Python: one device step
    at a time (th_llama_generate, 1 step, logits returned) and the oracle
    sampler on the device's own logits."""
    s = oracle.OracleSampler(seed=seed, stop_token=stop, **kw)
    m = device_llama(dev, cfg, 7, 8, prefill)
    past, out, tok = list(prompt), [], prompt[-1]
    try:
        for i in range(steps):
            _, logits = device_generate(m, cfg, tok, prefill + i, 1)
            nxt = s.sample(logits, past)
            if stop is not None and nxt == stop:
                break
            past.append(nxt)
            out.append(nxt)
            tok = nxt
    finally:
        capi.lib().th_llama_destroy(m)
    return out


def _device_sampled(dev, cfg, prompt, prefill, steps, seed, stop=None, **kw):
    m = device_llama(dev, cfg, 7, 8, prefill)
    s = capi.Sampler(capi.SamplingConfig(max_tokens=steps, stop_token=stop, **kw), seed=seed)
    try:
        pr = np.array(prompt, np.int32)
        out = np.empty(steps, np.int32)
        n = ctypes.c_size_t()
        capi.check(capi.lib().th_llama_generate_sampled(m, s.handle, capi.ptr(pr), pr.size, prefill, capi.ptr(out),
                                                        ctypes.byref(n)))
    finally:
        s.close()
        capi.lib().th_llama_destroy(m)
    return [int(t) for t in out[: n.value]]


def test_small_llama_sampled_generation(dev):
    """Non-greedy generate(): temperature, top-k, top-p and repetition
    penalty on the host, every step on the device.  A categorical draw is
    not a numerically stable function of the logits (a draw near a CDF
    boundary flips with a 1e-6 change), so the pins are: the sampler equals
    the oracle's on identical logits (test_sampling.py), the device logits
    equal the oracle's (tests above), and here th_llama_generate_sampled
    equals device steps fed through the oracle sampler, token for token,
    with the stop token ending the run before it is appended
    (sampling.rs:246-250)."""
    cfg = CONFIG_SMALL
    kw = dict(temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.1)
    prompt, prefill, steps = [3, 17, 1], 100, 24
    want = _device_steps_oracle_sampler(dev, cfg, prompt, prefill, steps, 11, **kw)
    got = _device_sampled(dev, cfg, prompt, prefill, steps, 11, **kw)
    print("composed", want)
    print("engine  ", got)
    assert got == want and len(got) == steps and len(set(got)) > 3
    stop = want[steps // 2]
    got_stop = _device_sampled(dev, cfg, prompt, prefill, steps, 11, stop=stop, **kw)
    assert got_stop == want[:want.index(stop)]


def _prefill(m, cfg, toks, pos):
    pr = np.array(toks, np.int32)
    nxt = ctypes.c_int32()
    logits = np.empty(cfg["vocab"], np.float32)
    capi.check(capi.lib().th_llama_prefill(m, capi.ptr(pr), pr.size, pos, ctypes.byref(nxt), capi.ptr(logits)))
    return nxt.value, logits


@pytest.mark.parametrize("n,hd", [(1, 64), (37, 64), (600, 64), (37, 256)])
def test_small_llama_prefill_matches_oracle(dev, n, hd):
    """th_llama_prefill (M=n GEMMs, causal attention, K/V appended) against
    the oracle fed the same tokens one decode step at a time: the last logits
    within the bf16-activation bar, the same next token, and 12 greedy decode
    steps continuing from the state prefill leaves (which read the K/V rows
    prefill wrote) match the oracle's continuation.  n=600 runs two prompt
    chunks; head_dim 64 takes the MFMA flash attention, 256 the split
    attention (one head of 256)."""
    cfg = dict(CONFIG_SMALL, max_seq=max(CONFIG_SMALL["max_seq"], 100 + n + 16))
    if hd != CONFIG_SMALL["head_dim"]:
        cfg.update(n_heads=CONFIG_SMALL["d_model"] // hd, n_kv_heads=1, head_dim=hd)
    prefill, steps = 100, 12
    print(f"prefill n={n} head_dim={hd}", flush=True)
    rng = np.random.default_rng(n)
    toks = [int(t) for t in rng.integers(0, cfg["vocab"], n)]
    ref = OracleLlama(cfg, 7, 8, prefill)
    for i, t in enumerate(toks):
        r_next, r_logits = ref.step(t, prefill + i)
    r_cont, _, _ = ref.generate(int(r_next), prefill + n, steps)
    m = device_llama(dev, cfg, 7, 8, prefill)
    try:
        nxt, logits = _prefill(m, cfg, toks, prefill)
        cont, _ = device_generate(m, cfg, nxt, prefill + n, steps)
    finally:
        capi.lib().th_llama_destroy(m)
    err = max_abs_rel(logits, r_logits)
    print("max_abs_rel", err, "next", nxt, int(r_next))
    assert err < 2e-2
    assert nxt == int(r_next)
    assert list(cont) == r_cont


@pytest.mark.parametrize("tied", [False, True])
def test_llama_from_safetensors_matches_oracle(dev, tmp_path, tied):
    """th_llama_load_safetensors (load_model, smollm.rs:364-420) on a small
    random model written with the safetensors package: f32 tensors, one f16
    tensor, and with `tied` no lm_head.weight (the embedding is reused).
    The oracle quantizes the same values with quantize_matrix_q4."""
    from safetensors.numpy import save_file

    cfg = CONFIG_SMALL
    L, d, ff, V = cfg["n_layers"], cfg["d_model"], cfg["d_ff"], cfg["vocab"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    rng = np.random.default_rng(5 + tied)
    shapes = {"self_attn.q_proj": (qd, d), "self_attn.k_proj": (kvd, d), "self_attn.v_proj": (kvd, d),
              "self_attn.o_proj": (d, qd), "mlp.gate_proj": (ff, d), "mlp.up_proj": (ff, d),
              "mlp.down_proj": (d, ff)}
    # a tied head reads the embedding: keep it small, or every step repeats the input token
    stored = {"model.embed_tokens.weight": rng.normal(0, 0.02 if tied else 0.5, (V, d)).astype(np.float32),
              "model.norm.weight": rng.normal(1, 0.1, d).astype(np.float32)}
    if not tied:
        stored["lm_head.weight"] = rng.normal(0, 0.05, (V, d)).astype(np.float32)
    for l in range(L):
        for name, shape in shapes.items():
            stored["model.layers.%d.%s.weight" % (l, name)] = rng.normal(0, 0.05, shape).astype(np.float32)
        stored["model.layers.%d.input_layernorm.weight" % l] = rng.normal(1, 0.1, d).astype(np.float32)
        stored["model.layers.%d.post_attention_layernorm.weight" % l] = rng.normal(1, 0.1, d).astype(np.float32)
    stored["model.layers.0.self_attn.q_proj.weight"] = stored["model.layers.0.self_attn.q_proj.weight"].astype(
        np.float16)
    # near-zero rows and a zero row: block scales below f16's normal range
    # (stored as f16 subnormals or zero) must load, not abort
    stored["model.layers.1.mlp.down_proj.weight"][:3] *= np.float32(1e-6)
    stored["model.layers.1.mlp.down_proj.weight"][3] = 0.0
    stored["model.layers.1.self_attn.v_proj.weight"][5, :64] *= np.float32(1e-4)
    path = tmp_path / "model.safetensors"
    save_file(stored, str(path))
    tensors = {k: v.astype(np.float32) for k, v in stored.items()}

    prefill, steps = 60, 24
    ref = OracleLlama(cfg, 0, 8, prefill, tensors=tensors)
    r_toks, margins, r_logits = ref.generate(1, prefill, steps)
    c = capi.LlamaConfig(L, d, cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], ff, V, cfg["max_seq"],
                         cfg["eps"], cfg["rope_theta"])
    m = ctypes.c_void_p()
    f = capi.SafetensorsFile(path)
    capi.check(capi.lib().th_llama_create(dev.handle, ctypes.byref(c), ctypes.byref(m)))
    try:
        capi.check(capi.lib().th_llama_load_safetensors(m, f.handle))
        capi.check(capi.lib().th_llama_fill_kv_synthetic(m, prefill, 8))
        toks, logits = device_generate(m, cfg, 1, prefill, steps)
    finally:
        capi.lib().th_llama_destroy(m)
        f.close()
    print("oracle", r_toks[:12], "min margin %.3e" % min(margins))
    print("device", list(toks[:12]))
    assert list(toks) == r_toks
    # bf16 activations: with O(1) norm weights a one-ulp bf16 difference at a
    # rounding point moves the logits by ~1e-3, so the bf16 bound applies
    assert max_abs_rel(logits, r_logits) < 2e-2


def test_llama_safetensors_rejects_missing_and_misshaped(dev, tmp_path):
    from safetensors.numpy import save_file

    cfg = CONFIG_SMALL
    c = capi.LlamaConfig(cfg["n_layers"], cfg["d_model"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                         cfg["d_ff"], cfg["vocab"], cfg["max_seq"], cfg["eps"], cfg["rope_theta"])
    path = tmp_path / "bad.safetensors"
    save_file({"model.embed_tokens.weight": np.zeros((3, 5), np.float32)}, str(path))
    f = capi.SafetensorsFile(path)
    m = ctypes.c_void_p()
    capi.check(capi.lib().th_llama_create(dev.handle, ctypes.byref(c), ctypes.byref(m)))
    try:
        with pytest.raises(capi.TangHipError):
            capi.check(capi.lib().th_llama_load_safetensors(m, f.handle))
    finally:
        capi.lib().th_llama_destroy(m)
        f.close()
