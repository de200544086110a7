"""Decode-engine parity: greedy tokens identical to the CPU oracle's.

Small config: compared live with the oracle (GQA, head_dim 64).
7B config: 128 greedy steps from position 2048 compared
with tests/golden/llama7b_decode.json, which tests/golden/make_decode_golden.py
wrote by running the oracle on the same seeded synthetic model.
"""
import json
import os

import numpy as np
import pytest

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


@pytest.mark.skipif(not os.path.exists(GOLDEN), reason="golden vectors not generated")
def test_7b_decode_128_steps_match_golden(dev):
    g = json.load(open(GOLDEN))
    cfg = CONFIG_7B
    m = device_llama(dev, cfg, g["seed"], g["kv_seed"], g["prefill"])
    try:
        toks, logits = device_generate(m, cfg, g["first_token"], g["prefill"], g["steps"])
    finally:
        capi.lib().th_llama_destroy(m)
    print("min oracle top-2 margin %.3e" % min(g["margins"]))
    mism = [i for i, (a, b) in enumerate(zip(toks, g["tokens"])) if a != b]
    print("first mismatches:", mism[:5])
    assert list(toks) == g["tokens"]
    last = np.array(g["last_logits_head"], np.float32)
    assert max_abs_rel(logits[: last.size], last) < 1e-3
