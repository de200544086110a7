"""Replay on the library's own AQL queue (tang_amd/csrc/aql.cpp) against HIP
launches of the same kernels: identical outputs, bit for bit.

The decode step and the benchmarked GEMV chain replay as AQL sequences with
no release fences between kernels (their kernels store what later kernels
read write-through); TANG_HIP_DISPATCH=graph switches the engine back to a
HIP graph, which a child process runs here for the comparison.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

from llama_ref import CONFIG_7B, CONFIG_SMALL, device_generate, device_llama
from tang_amd import capi

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("m", [1, 4, 16])
def test_q4_gemv_aql_chain_matches_stream(dev, m):
    """A 30-launch chain over three weight matrices (different values) on the
    AQL queue leaves the output of the last launch, as launches on the
    stream do."""
    print(f"aql gemv m={m}", flush=True)
    N, K = 1000, 2048
    ws = []
    for s in (5, 6, 7):
        nib, sc = capi.synth_q4(s, N, K)
        ws.append(dev.q4_upload_packed(nib, sc, N, K, capi.F16))
    x = dev.upload(capi.synth_normal(9, m * K, 1.0, capi.BF16), capi.BF16)
    y = dev.alloc(m * N)
    try:
        dev.bench_linear(x, m, ws, y, 30)
        ref = y.to_numpy().copy()
        for rep in range(2):
            y.upload(np.zeros(m * N, np.float32))
            ms = dev.bench_linear(x, m, ws, y, 30, use_graph="aql")
            assert ms > 0
            assert np.array_equal(y.to_numpy(), ref), rep
        # launch 29 reads ws[2]: a one-launch stream call on ws[2] agrees
        y2 = dev.alloc(m * N)
        dev.bench_linear(x, m, [ws[2]], y2, 1)
        assert np.array_equal(y2.to_numpy(), ref)
    finally:
        for w in ws:
            w.free()


def test_aql_sequence_longer_than_the_queue(dev):
    """One sequence of 5000 launches (the queue holds 4096 packets): the
    submission waits for ring space and wraps around the ring's end, and
    rings the doorbell at its last slot; the last launch's output equals the
    stream's."""
    N, K = 256, 512
    nib, sc = capi.synth_q4(21, N, K)
    ws = [dev.q4_upload_packed(nib, sc, N, K, capi.F16)]
    nib2, sc2 = capi.synth_q4(22, N, K)
    ws.append(dev.q4_upload_packed(nib2, sc2, N, K, capi.F16))
    x = dev.upload(capi.synth_normal(23, K, 1.0, capi.BF16), capi.BF16)
    y = dev.alloc(N)
    try:
        dev.bench_linear(x, 1, ws, y, 5000)
        ref = y.to_numpy().copy()
        for rep in range(2):
            y.upload(np.zeros(N, np.float32))
            dev.bench_linear(x, 1, ws, y, 5000, use_graph="aql")
            assert np.array_equal(y.to_numpy(), ref), rep
    finally:
        for w in ws:
            w.free()


def test_q8_gemv_aql_chain_matches_stream(dev):
    """The q8 GEMV chain (write-through outputs, no release fences) on the
    AQL queue: same outputs as on the stream."""
    q, rs = capi.synth_q8_rowwise(1, 512, 1024)
    ws = [dev.q8_upload_rowwise(q, rs, 512, 1024) for _ in range(2)]
    x = dev.upload(capi.synth_normal(11, 1024, 1.0, capi.F32))
    y = dev.alloc(512)
    try:
        dev.bench_linear(x, 1, ws, y, 8)
        ref = y.to_numpy().copy()
        y.upload(np.zeros(512, np.float32))
        dev.bench_linear(x, 1, ws, y, 8, use_graph="aql")
        assert np.array_equal(y.to_numpy(), ref)
    finally:
        for w in ws:
            w.free()


_CHILD = r"""
import sys, numpy as np
sys.path.insert(0, {here!r}); sys.path.insert(0, {root!r})
from llama_ref import CONFIG_7B, CONFIG_SMALL, device_generate, device_llama
from tang_amd import capi
cfg = {cfg}
dev = capi.HipComputeDevice(0)
m = device_llama(dev, cfg, {seed}, {kv_seed}, {prefill})
toks, logits = device_generate(m, cfg, {token}, {prefill}, {steps})
capi.lib().th_llama_destroy(m)
dev.close()
np.savez({out!r}, toks=toks, logits=logits)
"""


def _graph_replay_child(tmp_path, cfg_name, seed, kv_seed, prefill, token, steps, timeout):
    """The same generation in a child process with TANG_HIP_DISPATCH=graph
    (HIP graph replay, with the fences HIP puts between graph nodes)."""
    out = str(tmp_path / "graph.npz")
    env = dict(os.environ, TANG_HIP_DISPATCH="graph")
    code = _CHILD.format(here=HERE, root=os.path.dirname(HERE), out=out, cfg=cfg_name, seed=seed, kv_seed=kv_seed,
                         prefill=prefill, token=token, steps=steps)
    print("child: graph dispatch, %s, %d steps" % (cfg_name, steps), flush=True)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr[-2000:]
    return np.load(out)


def test_decode_aql_matches_hip_graph(dev, tmp_path):
    """48 greedy steps of the small model: tokens and final logits from the
    AQL replay (this process) equal the HIP graph replay's (a child process
    with TANG_HIP_DISPATCH=graph) bit for bit."""
    cfg = CONFIG_SMALL
    m = device_llama(dev, cfg, 7, 8, 100)
    try:
        toks, logits = device_generate(m, cfg, 1, 100, 48)
        ms = ctypes.c_float()
        capi.check(capi.lib().th_llama_time_steps(m, 1, 100, 4, ctypes.byref(ms)))
        assert 0 < ms.value < 1e4
    finally:
        capi.lib().th_llama_destroy(m)
    g = _graph_replay_child(tmp_path, "CONFIG_SMALL", 7, 8, 100, 1, 48, 100)
    assert np.array_equal(g["toks"], toks)
    assert np.array_equal(g["logits"], logits)


def test_decode_7b_aql_matches_hip_graph(dev, tmp_path):
    """The 7B shape (config 3: 161 write-through kernels per step, attention
    split over every CU, workgroups on all eight XCDs), 6 greedy steps from
    position 2048: the AQL replay's tokens and final logits equal the HIP
    graph replay's bit for bit, so no kernel of the step reads a value
    another XCD left in its own L2."""
    cfg = CONFIG_7B
    m = device_llama(dev, cfg, 3, 33, 2048)
    try:
        toks, logits = device_generate(m, cfg, 10, 2048, 6)
    finally:
        capi.lib().th_llama_destroy(m)
    g = _graph_replay_child(tmp_path, "CONFIG_7B", 3, 33, 2048, 10, 6, 110)
    assert np.array_equal(g["toks"], toks)
    assert np.array_equal(g["logits"], logits)


def test_device_steps_continue_like_generate(dev):
    """th_llama_set_token + two th_llama_step_device calls (each one replay,
    the token chained on the device) leave the KV cache as th_llama_generate
    does: a one-step generate from there gives the same token and the same
    logits, bit for bit, as an uninterrupted three-step generate."""
    cfg = CONFIG_SMALL
    L = capi.lib()
    m = device_llama(dev, cfg, 7, 8, 100)
    try:
        ref_toks, ref_logits = device_generate(m, cfg, 1, 100, 3)
        capi.check(L.th_llama_fill_kv_synthetic(m, 100, 8))
        capi.check(L.th_llama_set_token(m, 1))
        capi.check(L.th_llama_step_device(m, 100))
        capi.check(L.th_llama_step_device(m, 101))
        toks, logits = device_generate(m, cfg, int(ref_toks[1]), 102, 1)
    finally:
        L.th_llama_destroy(m)
    assert int(toks[0]) == int(ref_toks[2])
    assert np.array_equal(logits, ref_logits)
