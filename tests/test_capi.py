"""CPU-side checks of the C-ABI library: it loads, exports every declared
entry point, validates arguments without a GPU, and its host-side helpers
(synthetic generators, RoPE tables) are deterministic and match the oracle."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from tang_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tang_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(th_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(capi.LIB_PATH)
    names = declared_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(declared_symbols()) == set(capi.SIGNATURES)


def test_null_arguments_are_errors_not_crashes():
    L = capi.lib()
    assert L.th_device_create(0, None) == capi.TH_ERR_INVALID
    assert b"null" in L.th_last_error()
    assert L.th_gemm_q4(None, None, 1, None, None) == capi.TH_ERR_INVALID
    assert L.th_kv_attention(None, None, None, None, 0, 1, 1, 1, 1, None) == capi.TH_ERR_INVALID
    assert L.th_buffer_free(None) == capi.TH_OK


def test_synth_is_deterministic_and_distributed():
    nib, sc = capi.synth_q4(123, 64, 4096)
    nib2, sc2 = capi.synth_q4(123, 64, 4096)
    assert np.array_equal(nib, nib2) and np.array_equal(sc, sc2)
    vals = np.concatenate([(nib & 15).ravel(), (nib >> 4).ravel()]).astype(np.int64) - 8
    assert vals.min() == -8 and vals.max() == 7
    counts = np.bincount(vals + 8, minlength=16)
    assert counts.min() > 0.9 * counts.mean()
    s = sc.view(np.float16).astype(np.float32)
    assert s.min() >= 0.002 - 1e-6 and s.max() <= 0.01 + 1e-5
    q, rs = capi.synth_q8_rowwise(5, 32, 256)
    assert q.min() >= -127 and q.max() <= 127 and rs.min() >= 0.005 and rs.max() <= 0.02
    z = capi.synth_normal(9, 200000, 1.0, capi.F32)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    zb = capi.synth_normal(9, 1000, 1.0, capi.BF16)
    assert np.array_equal(zb, oracle.f32_to_bf16(z[:1000]))
    zh = capi.synth_normal(9, 1000, 1.0, capi.F16)
    assert np.array_equal(zh, oracle.f32_to_f16(z[:1000]))


def test_synth_ragged_tail_is_zero_weight():
    nib, _ = capi.synth_q4(7, 3, 40)  # 2 blocks, 8 live elements in the second
    tail = nib[:, 16 + 4:]
    assert np.all(tail == 0x88)


def test_rope_tables_match_oracle_bitwise():
    c, s = capi.rope_tables(128, 300, 10000.0)
    oc, os_ = oracle.rope_tables(128, 300, 10000.0)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)


def test_seed_mixing_distinct():
    seeds = {capi.synth_seed(3, l, t) for l in range(32) for t in range(8)}
    assert len(seeds) == 256
