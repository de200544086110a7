"""MoE layer against the oracle's from-definition MoE.
Routing (top-k indices) must match exactly; the outputs within 2e-2
max-abs-rel (bf16 activations)."""
import numpy as np
import pytest

from conftest import max_abs_rel
from moe_ref import CONFIG4, OracleMoe, device_moe, device_moe_forward
from tang_amd import capi

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [1, 16, 40, 64, 65, 100, 257, 512])  # > 64 tokens: grouped MFMA GEMM; 512: config 4 prefill
def test_moe_matches_oracle(dev, T):
    cfg = CONFIG4
    print(f"moe T={T}", flush=True)
    h = capi.synth_normal(41 + T, T * cfg["d"], 1.0, capi.BF16)
    ref = OracleMoe(cfg, 4)
    r_out, r_idx, r_w = ref.forward(h, T)
    m = device_moe(dev, cfg, 4)
    try:
        out, idx, w = device_moe_forward(dev, m, cfg, h, T)
    finally:
        capi.lib().th_moe_destroy(m)
    assert np.array_equal(idx, r_idx)
    assert max_abs_rel(w, r_w) < 1e-5
    err = max_abs_rel(out, r_out)
    print("max_abs_rel", err)
    assert err < 2e-2


def test_moe_small_shape_and_repeat(dev):
    """Odd sizes (d=256, ff=96, 8 experts, 1 shared, top-3) and two calls on
    one instance (work buffers reused, counters reset)."""
    cfg = dict(d=256, ff=96, E=8, S=1, k=3)
    ref = OracleMoe(cfg, 9)
    m = device_moe(dev, cfg, 9)
    try:
        for T in (5, 33):
            h = capi.synth_normal(T, T * cfg["d"], 1.0, capi.BF16)
            r_out, r_idx, _ = ref.forward(h, T)
            out, idx, _ = device_moe_forward(dev, m, cfg, h, T)
            assert np.array_equal(idx, r_idx)
            assert max_abs_rel(out, r_out) < 2e-2
    finally:
        capi.lib().th_moe_destroy(m)


def test_moe_tied_router_logits(dev):
    """A zero hidden state gives every expert the same logit: top-k must take
    experts 0..k-1 in index order (first maximum on ties,
    sampling.rs:184-194), each with probability 1/E."""
    cfg = dict(d=256, ff=96, E=8, S=1, k=3)
    T = 4
    h = np.zeros(T * cfg["d"], np.uint16)  # bf16 zeros
    ref = OracleMoe(cfg, 9)
    r_out, r_idx, r_w = ref.forward(h, T)
    m = device_moe(dev, cfg, 9)
    try:
        out, idx, w = device_moe_forward(dev, m, cfg, h, T)
    finally:
        capi.lib().th_moe_destroy(m)
    expect = np.tile(np.arange(cfg["k"], dtype=np.int32), (T, 1))
    assert np.array_equal(r_idx, expect) and np.array_equal(idx, expect)
    assert np.allclose(w, 1.0 / cfg["E"], rtol=0, atol=1e-7)
    assert max_abs_rel(out, r_out) < 2e-2


@pytest.mark.parametrize("T", [20, 70])  # top-k inside the dispatch kernel / in its own kernel
def test_moe_many_experts(dev, T):
    """100 routed experts, no shared one: two expert slots per lane in the
    top-k and a probability row that is not a whole number of 16-float
    rounds."""
    cfg = dict(d=256, ff=64, E=100, S=0, k=6)
    print(f"moe E=100 T={T}", flush=True)
    h = capi.synth_normal(7 + T, T * cfg["d"], 1.0, capi.BF16)
    ref = OracleMoe(cfg, 11)
    r_out, r_idx, r_w = ref.forward(h, T)
    m = device_moe(dev, cfg, 11)
    try:
        out, idx, w = device_moe_forward(dev, m, cfg, h, T)
    finally:
        capi.lib().th_moe_destroy(m)
    assert np.array_equal(idx, r_idx)
    assert max_abs_rel(w, r_w) < 1e-5
    assert max_abs_rel(out, r_out) < 2e-2


@pytest.mark.parametrize("T", [6, 80])  # grouped GEMV / grouped MFMA GEMM
def test_moe_many_shared_experts(dev, T):
    """Ten shared experts (more than one load round of the combine) and a
    top-9 routing (more than eight ranks per token)."""
    cfg = dict(d=256, ff=64, E=16, S=10, k=9)
    print(f"moe S=10 k=9 T={T}", flush=True)
    h = capi.synth_normal(90 + T, T * cfg["d"], 1.0, capi.BF16)
    ref = OracleMoe(cfg, 13)
    r_out, r_idx, _ = ref.forward(h, T)
    m = device_moe(dev, cfg, 13)
    try:
        out, idx, _ = device_moe_forward(dev, m, cfg, h, T)
    finally:
        capi.lib().th_moe_destroy(m)
    assert np.array_equal(idx, r_idx)
    assert max_abs_rel(out, r_out) < 2e-2


@pytest.mark.parametrize("T", [16, 100])  # grouped GEMV and grouped MFMA GEMM
def test_moe_graph_replay_matches_eager(dev, T):
    """Two forward calls on different hidden states recorded into one HIP
    graph (th_capture_begin / th_capture_end) and replayed three times, with
    eager calls and synchronisations between the replays: every replay gives
    the eager outputs and routing bit for bit (the routing counters and work
    lists are rebuilt in-graph on every replay)."""
    import ctypes
    cfg = CONFIG4
    L = capi.lib()
    m = device_moe(dev, cfg, 4)
    try:
        hs = [dev.upload(capi.synth_normal(s, T * cfg["d"], 1.0, capi.BF16), capi.BF16) for s in (7, 8)]
        outs = [dev.alloc(T * cfg["d"]) for _ in hs]
        idxs = [dev.alloc(T * cfg["k"], capi.I32) for _ in hs]
        ws = [dev.alloc(T * cfg["k"]) for _ in hs]

        def both():
            for i in range(2):
                capi.check(L.th_moe_forward(m, hs[i].handle, T, outs[i].handle, idxs[i].handle, ws[i].handle))

        both()
        dev.sync()
        eager = [(o.to_numpy().copy(), x.to_numpy().copy(), w.to_numpy().copy()) for o, x, w in zip(outs, idxs, ws)]
        g = dev.capture(both)
        try:
            for rep in range(3):
                for o in outs:
                    o.upload(np.zeros(T * cfg["d"], np.float32))
                g.launch()
                dev.sync()
                for i in range(2):
                    assert np.array_equal(outs[i].to_numpy(), eager[i][0]), (rep, i)
                    assert np.array_equal(idxs[i].to_numpy(), eager[i][1]), (rep, i)
                    assert np.array_equal(ws[i].to_numpy(), eager[i][2]), (rep, i)
                capi.check(L.th_moe_forward(m, hs[1].handle, T, outs[0].handle, idxs[0].handle, ws[0].handle))
                dev.sync()  # eager work between replays
        finally:
            g.free()
    finally:
        L.th_moe_destroy(m)
