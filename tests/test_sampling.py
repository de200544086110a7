"""Sampling beyond greedy (crates/tang-infer/src/sampling.rs): the product's
host sampler (C ABI, sampling.cpp) and the oracle's C restatement, both run
on the CPU.  Pinned by the reference's own tests (sampling.rs:263-430) and by
the two restatements agreeing token for token on random logits, ties and
every filter combination."""
import numpy as np
import pytest

import oracle
from tang_amd import capi


def _both(**kw):
    seed = kw.pop("seed", 42)
    return (oracle.OracleSampler(seed=seed, **kw),
            capi.Sampler(capi.SamplingConfig(**kw), seed=seed))


@pytest.mark.parametrize("which", [0, 1])
def test_reference_greedy_kats(which):  # sampling.rs:263-300
    s = _both(temperature=0.0)[which]
    assert s.sample([1.0, 3.0, 10.0, 2.0]) == 2
    for _ in range(10):
        assert s.sample([1.0, 5.0, 3.0]) == 1
    assert s.sample([1.0, 2.0, 5.0, 3.0]) == 2


@pytest.mark.parametrize("which", [0, 1])
def test_reference_top_k_kat(which):  # sampling.rs:302-326
    s = _both(temperature=1.0, top_k=2, top_p=1.0, seed=12345)[which]
    seen = {s.sample([1.0, 100.0, 0.1, 99.0]) for _ in range(100)}
    assert seen == {1, 3}


@pytest.mark.parametrize("which", [0, 1])
def test_reference_top_p_kat(which):  # sampling.rs:328-339
    s = _both(temperature=1.0, top_k=0, top_p=0.5, seed=99)[which]
    assert all(s.sample([10.0, 0.0, 0.0, 0.0]) == 0 for _ in range(20))


@pytest.mark.parametrize("which", [0, 1])
def test_reference_repetition_penalty_kat(which):  # sampling.rs:341-357
    s = _both(temperature=0.0, repetition_penalty=100.0)[which]
    assert s.sample([5.0, 4.9, 4.8], past=[0]) == 1


@pytest.mark.parametrize("which", [0, 1])
def test_reference_temperature_variety_kat(which):  # sampling.rs:405-428
    s = _both(temperature=2.0, seed=777)[which]
    assert len({s.sample([1.0, 1.0, 1.0, 1.0]) for _ in range(100)}) >= 3


def test_lcg_draw_matches_closed_form():
    """Uniform logits over n tokens: the token is the first i with
    r < (i+1)/n summed in f64, r from the LCG of sampling.rs:77-80."""
    state = 2024
    a, c = 6364136223846793005, 1442695040888963407
    s = _both(temperature=1.0, seed=2024)
    n = 7
    for _ in range(50):
        state = (state * a + c) % (1 << 64)
        r = (state >> 11) / float(1 << 53)
        cum, want = 0.0, n - 1
        for i in range(n):
            cum += 1.0 / n
            if r < cum:
                want = i
                break
        assert s[0].sample(np.zeros(n)) == want
        assert s[1].sample(np.zeros(n)) == want


@pytest.mark.parametrize("temperature", [0.0, 0.7, 1.0, 1.6])
@pytest.mark.parametrize("top_k", [0, 1, 5, 40])
@pytest.mark.parametrize("top_p", [1.0, 0.9, 0.3])
def test_product_matches_oracle(temperature, top_k, top_p):
    rng = np.random.default_rng(int(temperature * 10) + 100 * top_k + int(top_p * 1000))
    o, d = _both(temperature=temperature, top_k=top_k, top_p=top_p, repetition_penalty=1.3, seed=5)
    past = []
    for step in range(40):
        logits = rng.normal(0, 3, 997).astype(np.float32)
        if step % 3 == 0:  # ties: few distinct values exercise the stable orders and the k-th threshold
            logits = np.round(logits).astype(np.float32)
        a, b = o.sample(logits, past), d.sample(logits, past)
        assert a == b, (step, a, b)
        past.append(a)


def test_sampler_rejects_bad_config():
    with pytest.raises(capi.TangHipError):
        capi.Sampler(capi.SamplingConfig(temperature=-1.0))
