"""Headline benchmark: int4 group-32 GEMV HBM bandwidth (
11008x4096, M=1, bf16 activations) plus the 7B-shape int4 batch-1 decode rate
(config 3), on one MI355X; also config 1 (int8 GEMV), config 4 (MoE),
config 5 (MLA) and the prefill GEMM as secondary sections.

One "step" is one GEMV launch over one batch (M=1) of synthetic activations.
The timed loop cycles through enough distinct weight copies (>256 MiB) that
the weights stream from HBM, not the 256 MB Infinity Cache.  Times come from
HIP events recorded on the library's own stream (th_bench_linear,
th_llama_time_steps).  The CPU baseline is the oracle's restatement of the
reference q4_matvec (crates/tang-infer/src/quantize.rs:256-289), f64,
single thread, on a bounded sample of the same workload
(`cpu_baseline`), and the same restatement on every other config, one core
and all cores (`cpu_baselines_all_configs`, with the CPU model and nproc).

Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from tang_amd import capi  # noqa: E402

METRIC = "Q4 GEMV HBM GB/s (% of peak); decode tok/s, 7B-shape int4, batch 1"
PEAK_HBM_GBS = 8000.0
N, K = 11008, 4096
GEMV_BYTES = {1: 25414656, 4: 25571328, 8: 25780224, 16: 26198016}  # algorithmic bytes per call
N_COPIES = 12  # 12 x 25.4 MB = 305 MB > 256 MB last-level cache
# HBM bytes per M=1 launch from the rocprofv3 FETCH_SIZE + WRITE_SIZE runs in
# profiles/q4_gemv_config2.md, each scaled by its reading of a known-size copy.
TRAFFIC_BYTES = 25547776

CFG7B = dict(n_layers=32, d_model=4096, n_heads=32, n_kv_heads=32, head_dim=128, d_ff=11008, vocab=32000,
             max_seq=2176, eps=1e-5, rope_theta=1e4)


def gemv_bench(dev, m, steps, warmup, graph="aql"):
    """Elapsed ms of `steps` config-2 linears over N_COPIES weight copies;
    graph="aql" replays them as one sequence on the library's AQL queue (the
    decode engine's launch mode: no release fences between the launches),
    True as one HIP graph, False launches each on the stream."""
    nib, sc16 = capi.synth_q4(2, N, K)
    ws = [dev.q4_upload_packed(nib, sc16, N, K, capi.F16) for _ in range(N_COPIES)]
    x = dev.upload(capi.synth_normal(3, m * K, 1.0, capi.BF16), capi.BF16)
    y = dev.alloc(m * N)
    if warmup:
        dev.bench_linear(x, m, ws, y, warmup)
    if graph == "aql":  # the whole protocol once, untimed: the first AQL replays of a process run slow
        dev.bench_linear(x, m, ws, y, steps, use_graph=graph)
    ms = dev.bench_linear(x, m, ws, y, steps, use_graph=graph)
    for w in ws:
        w.free()
    return ms


Q8_BYTES = 4096 * 4096 + 3 * 4096 * 4  # config 1: W, row scales, x, y


def q8_bench(dev, steps, copies=18):
    """Config 1: int8 4096x4096 GEMV, per-row scales, f32 x (18 copies =
    302 MB > MALL), replayed as one sequence on the library's AQL queue."""
    q, rs = capi.synth_q8_rowwise(1, 4096, 4096)
    ws = [dev.q8_upload_rowwise(q, rs, 4096, 4096) for _ in range(copies)]
    x = dev.upload(capi.synth_normal(11, 4096, 1.0, capi.F32))
    y = dev.alloc(4096)
    dev.bench_linear(x, 1, ws, y, 48)
    dev.bench_linear(x, 1, ws, y, steps, use_graph="aql")  # the protocol once, untimed
    ms = dev.bench_linear(x, 1, ws, y, steps, use_graph="aql")
    for w in ws:
        w.free()
    us = ms * 1e3 / steps
    return dict(workload="q8 per-row GEMV 4096x4096, M=1, f32 activations (BASELINE config 1)", us=round(us, 3),
                gbs=round(Q8_BYTES / us / 1e3, 1), frac_hbm=round(Q8_BYTES / us / 1e3 / PEAK_HBM_GBS, 4))


PEAK_BF16_TFLOPS = 2500.0


def prefill_bench(dev, m, steps=30):
    """Prefill-shaped int4 GEMM on the config-2 matrix: MFMA path."""
    nib, sc16 = capi.synth_q4(2, N, K)
    ws = [dev.q4_upload_packed(nib, sc16, N, K, capi.F16) for _ in range(3)]
    x = dev.upload(capi.synth_normal(3, m * K, 1.0, capi.BF16), capi.BF16)
    y = dev.alloc(m * N)
    dev.bench_linear(x, m, ws, y, 3)
    ms = dev.bench_linear(x, m, ws, y, steps, use_graph=True)
    for w in ws:
        w.free()
    us = ms * 1e3 / steps
    tf = 2.0 * m * N * K / us / 1e6
    return dict(M=m, us=round(us, 1), tflops=round(tf, 1), frac_mfma_bf16=round(tf / PEAK_BF16_TFLOPS, 4))


def blas_reference():
    """The library's plain dense GEMM (torch.matmul on ROCm: hipBLASLt) on the
    prefill GEMM shapes, as a reference point for the MFMA rate this part
    sustains on random and on constant operands.  Not part of the bench line."""
    import torch
    out = []
    dev = torch.device("cuda:0")
    for dt, name in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        for m in (512, 2048):
            for fill in ("randn", "ones"):
                if fill == "ones" and (dt != torch.float16 or m != 2048):
                    continue
                mk = torch.randn if fill == "randn" else torch.ones
                a, b = mk(m, K, dtype=dt, device=dev), mk(N, K, dtype=dt, device=dev)
                for _ in range(5):
                    a @ b.t()
                torch.cuda.synchronize()
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                for _ in range(50):
                    a @ b.t()
                e.record()
                torch.cuda.synchronize()
                us = s.elapsed_time(e) * 1e3 / 50
                out.append(dict(dtype=name, M=m, operands=fill, us=round(us, 1),
                                tflops=round(2.0 * m * N * K / us / 1e6, 1)))
    return {"blas_reference": out, "shape": "M x 4096 times (11008 x 4096)^T"}


def decode_bytes_per_token(c, t_attended):
    """Algorithmic HBM bytes of one decode step: every weight byte, the KV
    rows attended, norms and one embedding row, each counted once."""
    d, ff, L, V = c["d_model"], c["d_ff"], c["n_layers"], c["vocab"]
    kvd = c["n_kv_heads"] * c["head_dim"]
    qd = c["n_heads"] * c["head_dim"]
    lin = L * (d * (qd + 2 * kvd) + qd * d + 2 * d * ff + ff * d) + V * d
    weights = lin // 2 + (lin // 32) * 2
    kv = L * 2 * t_attended * kvd * 2
    return weights + kv + (2 * L + 1) * d * 2 + d * 2


def decode_bench(dev, steps):
    import ctypes
    c = CFG7B
    cfg = capi.LlamaConfig(c["n_layers"], c["d_model"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["d_ff"],
                           c["vocab"], c["max_seq"], c["eps"], c["rope_theta"])
    L = capi.lib()
    h = ctypes.c_void_p()
    t0 = time.time()
    capi.check(L.th_llama_create(dev.handle, ctypes.byref(cfg), ctypes.byref(h)))
    try:
        capi.check(L.th_llama_init_synthetic(h, 3))
        capi.check(L.th_llama_fill_kv_synthetic(h, 2048, 33))
        init_s = time.time() - t0
        ms = ctypes.c_float()
        capi.check(L.th_llama_time_steps(h, 10, 2048, 8, ctypes.byref(ms)))  # warm (records the step)
        capi.check(L.th_llama_fill_kv_synthetic(h, 2048, 33))
        capi.check(L.th_llama_time_steps(h, 10, 2048, steps, ctypes.byref(ms)))
        pf = prefill_7b(L, h, c)
    finally:
        L.th_llama_destroy(h)
    per_tok_ms = ms.value / steps
    mean_bytes = np.mean([decode_bytes_per_token(c, 2049 + i) for i in range(steps)])
    roof_tok_s = PEAK_HBM_GBS * 1e9 / mean_bytes
    tok_s = 1e3 / per_tok_ms
    return dict(tok_s=round(tok_s, 1), ms_per_token=round(per_tok_ms, 4), steps=steps,
                bytes_per_token_mean=int(mean_bytes), roofline_tok_s=round(roof_tok_s, 1),
                frac_of_roofline=round(tok_s / roof_tok_s, 4), kv_positions="2049..%d" % (2048 + steps),
                init_s=round(init_s, 1), prefill=pf)


def prefill_7b(L, h, c, n=512):
    """th_llama_prefill of an n-token prompt at positions 0..n-1 (M=n int4
    GEMMs on MFMA plus causal split attention), HIP events."""
    import ctypes
    toks = np.random.default_rng(0).integers(0, c["vocab"], n).astype(np.int32)
    ms = ctypes.c_float()
    capi.check(L.th_llama_time_prefill(h, capi.ptr(toks), n, 0, ctypes.byref(ms)))
    d, ff, Ln = c["d_model"], c["d_ff"], c["n_layers"]
    kvd = c["n_kv_heads"] * c["head_dim"]
    lin = Ln * (d * (d + 2 * kvd) + d * d + 2 * d * ff + ff * d)
    flops = 2.0 * n * lin + Ln * 2 * 2 * (n * (n + 1) / 2) * d  # linears + causal QK^T and PV
    us = ms.value * 1e3
    return dict(prompt_tokens=n, ms=round(ms.value, 2), tok_s=round(n / ms.value * 1e3, 1),
                tflops=round(flops / us / 1e6, 1), frac_mfma_bf16=round(flops / us / 1e6 / PEAK_BF16_TFLOPS, 4))


MOE = dict(d=2048, ff=1408, E=64, S=2, k=6)
MLA = dict(B=8, H=16, L=4096, dn=128, dr=64, r=512, dv=128)


def moe_bench(dev, T, iters, layers=2, graph=True):
    """Config 4 MoE layer forward (router, dispatch, grouped int4 experts,
    combine) on T tokens.  `layers` independently initialised layers are
    called in turn, so every call's expert weights were last read a whole
    layer earlier (2 x 321 MB > 256 MB MALL).  Algorithmic bytes per call:
    every weight byte of the experts the batch routes to (+ shared experts)
    once, the router, h in, out (averaged over the layers).  `us`: the calls
    replayed as one HIP graph (th_capture);
    `stream_launched_us`: the same calls enqueued one by one."""
    import ctypes
    c = MOE
    L = capi.lib()
    hs = []
    try:
        for i in range(layers):
            h = ctypes.c_void_p()
            capi.check(L.th_moe_create(dev.handle, c["d"], c["ff"], c["E"], c["S"], c["k"], ctypes.byref(h)))
            hs.append(h)
            capi.check(L.th_moe_init_synthetic(h, 4 + 100 * i))
        x = dev.upload(capi.synth_normal(45, T * c["d"], 1.0, capi.BF16), capi.BF16)
        out = dev.alloc(T * c["d"])
        idx = [dev.alloc(T * c["k"], capi.I32) for _ in hs]
        w = [dev.alloc(T * c["k"]) for _ in hs]
        fwd = lambda i: capi.check(L.th_moe_forward(hs[i % layers], x.handle, T, out.handle, idx[i % layers].handle,
                                                    w[i % layers].handle))
        for i in range(2 * layers):
            fwd(i)
        dev.sync()
        dev.timer_start()
        for i in range(iters):
            fwd(i)
        ms_stream = dev.timer_stop()
        ms = ms_stream
        if graph:
            g = dev.capture(lambda: [fwd(i) for i in range(iters)])
            g.launch()
            dev.timer_start()
            g.launch()
            ms = dev.timer_stop()
            g.free()
        used = [len(np.unique(b.to_numpy())) + c["S"] for b in idx]
    finally:
        for h in hs:
            L.th_moe_destroy(h)
    lin = 3 * c["ff"] * c["d"]
    nbytes = np.mean(used) * (lin // 2 + lin // 32 * 2) + c["E"] * c["d"] * 4 + T * c["d"] * (2 + 4)
    us = ms * 1e3 / iters
    flops = 2 * T * (c["k"] + c["S"]) * lin
    return dict(T=T, us=round(us, 2), experts_read=used, bytes=int(nbytes), gbs=round(nbytes / us / 1e3, 1),
                frac_hbm=round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), tflops=round(flops / us / 1e6, 2),
                stream_launched_us=round(ms_stream * 1e3 / iters, 2), layers_rotated=layers)


def mla_bench(dev, iters, copies=8):
    """Config 5 absorbed MLA decode, B=8 sequences x 4096 latent positions.
    Rotates `copies` caches (8 x 37.7 MB > 256 MB MALL).  Algorithmic bytes:
    the latent cache, W_UK and W_UV with their scales, q in, out.  `us`: the
    calls replayed as one HIP graph; `stream_launched_us`: enqueued one by one."""
    c = MLA
    B, H, Lk, dn, dr, r, dv = c["B"], c["H"], c["L"], c["dn"], c["dr"], c["r"], c["dv"]
    qn = dev.upload(capi.synth_normal(1, B * H * dn, 1.0, capi.F32))
    qr = dev.upload(capi.synth_normal(2, B * H * dr, 1.0, capi.F32))
    host_cache = capi.synth_normal(3, B * Lk * (r + dr), 1.0, capi.BF16)
    caches = [dev.upload(host_cache, capi.BF16) for _ in range(copies)]
    wuk = dev.q8_upload_rowwise(*capi.synth_q8_rowwise(4, H * r, dn), H * r, dn)
    wuv = dev.q8_upload_rowwise(*capi.synth_q8_rowwise(5, H * dv, r), H * dv, r)
    out = dev.alloc(B * H * dv)
    scale = 1.0 / np.sqrt(dn + dr)
    for i in range(copies):
        dev.mla_decode(qn, qr, caches[i], B, H, Lk, dn, dr, r, dv, wuk, wuv, scale, out)
    dev.sync()
    call = lambda i: dev.mla_decode(qn, qr, caches[i % copies], B, H, Lk, dn, dr, r, dv, wuk, wuv, scale, out)
    dev.timer_start()
    for i in range(iters):
        call(i)
    ms_stream = dev.timer_stop()
    g = dev.capture(lambda: [call(i) for i in range(iters)])
    g.launch()
    dev.timer_start()
    g.launch()
    ms = dev.timer_stop()
    g.free()
    us = ms * 1e3 / iters
    nbytes = B * Lk * (r + dr) * 2 + H * r * (dn + 4) + H * dv * (r + 4) + B * H * (dn + dr + dv) * 4
    for b in caches:
        b.free()
    return dict(us=round(us, 2), bytes=int(nbytes), gbs=round(nbytes / us / 1e3, 1),
                frac_hbm=round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4), stream_launched_us=round(ms_stream * 1e3 / iters, 2))


def cpu_baseline(budget_s=12.0, threads=1):
    """Oracle q4_matvec (f64, the reference's serial per-row order) on
    config-2 rows: a bounded sample.  threads=1 is the faithful single-core
    restatement; threads>1 runs rows in parallel (OpenMP), each row's sum
    still serial."""
    import oracle
    nib, sc16 = capi.synth_q4(2, N, K)
    sc = oracle.f16_to_f32(sc16)
    x = oracle.bf16_to_f32(capi.synth_normal(3, K, 1.0, capi.BF16)).astype(np.float64)
    rows = 1376 if threads == 1 else N  # 1/8 of the matrix per call, or all of it
    calls, t0 = 0, time.time()
    while time.time() - t0 < budget_s:
        r0 = (calls * rows) % N
        oracle.q4_matvec_soa(nib[r0:r0 + rows], sc[r0:r0 + rows], rows, K, x, threads=threads)
        calls += 1
    dt = time.time() - t0
    full_calls = calls * rows / N
    us = dt / full_calls * 1e6
    return dict(value=round(GEMV_BYTES[1] / us / 1e3, 3), unit="GB/s", cores=threads, kind="port",
                sample="%d calls of q4_matvec on %d of the %d rows (%.1f s, %.0f us per full 11008x4096 call)"
                       % (calls, rows, N, dt, us))


def _timed(fn, budget_s, min_calls=1):
    """Calls fn until budget_s has passed (at least min_calls); seconds per call."""
    calls, t0 = 0, time.time()
    while calls < min_calls or time.time() - t0 < budget_s:
        fn()
        calls += 1
    return (time.time() - t0) / calls, calls


def cpu_config1(threads):
    """Config 1 on the oracle's q8_matvec (f64, serial per row)."""
    import oracle
    q, rs = capi.synth_q8_rowwise(1, 4096, 4096)
    x = capi.synth_normal(11, 4096, 1.0, capi.F32).astype(np.float64)
    scales = np.repeat(rs[:, None], 128, axis=1)
    sec, calls = _timed(lambda: oracle.q8_matvec_soa(q, scales, 4096, 4096, x, threads=threads), 3.0)
    return dict(us_per_call=round(sec * 1e6, 1), cores=threads, sample="%d full calls" % calls)


def cpu_config3(threads_all):
    """Config 3 decode step on the oracle (or_llama_decode_step): the whole
    32-layer 7B-shape model, KV prefilled to 2048, one greedy step at
    position 2048 timed on 1 thread (the reference is serial) and one on
    `threads_all` threads.  Each step appends its K/V row at 2048 again,
    so both time the same work."""
    from oracle.models import CONFIG_7B, OracleLlama
    t0 = time.time()
    ref = OracleLlama(CONFIG_7B, 3, 33, 2048, workers=threads_all)
    init_s = time.time() - t0
    out = []
    for threads in (1, threads_all):
        t0 = time.time()
        ref.step(10, 2048, threads=threads)
        dt = time.time() - t0
        out.append(dict(s_per_token=round(dt, 3), cores=threads,
                        sample="one full 32-layer step at position 2048 (weights generated in %.0f s, untimed)"
                               % init_s))
    del ref
    return out


def cpu_config4(threads, T, sample_tokens):
    """Config 4 MoE layer on the oracle (or_moe_forward, per token
    independent): sample_tokens of the T-token batch, scaled to T."""
    from oracle.models import CONFIG4, OracleMoe
    ref = OracleMoe(CONFIG4, 4)
    h = capi.synth_normal(45, sample_tokens * CONFIG4["d"], 1.0, capi.BF16)
    sec, calls = _timed(lambda: ref.forward(h, sample_tokens, threads=threads), 2.0)
    return dict(T=T, us_per_call=round(sec * T / sample_tokens * 1e6, 1), cores=threads,
                sample="%d calls on %d of the %d tokens" % (calls, sample_tokens, T))


def cpu_config5(threads):
    """Config 5 absorbed MLA decode on the oracle (or_mla_decode), B=8 x
    4096 positions."""
    import oracle
    c = MLA
    B, H, Lk, dn, dr, r, dv = c["B"], c["H"], c["L"], c["dn"], c["dr"], c["r"], c["dv"]
    qn = capi.synth_normal(1, B * H * dn, 1.0, capi.F32)
    qr = capi.synth_normal(2, B * H * dr, 1.0, capi.F32)
    cache = capi.synth_normal(3, B * Lk * (r + dr), 1.0, capi.BF16)
    wuk, suk = capi.synth_q8_rowwise(4, H * r, dn)
    wuv, suv = capi.synth_q8_rowwise(5, H * dv, r)
    sec, calls = _timed(lambda: oracle.mla_decode(qn, qr, cache, B, H, Lk, dn, dr, r, dv, wuk, suk, wuv, suv,
                                                  1.0 / np.sqrt(dn + dr), threads=threads), 2.0)
    return dict(us_per_call=round(sec * 1e6, 1), cores=threads, sample="%d full calls" % calls)


def cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name, vendor, family,
    model and stepping of the first processor, and the logical CPU count."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break  # the first processor's block
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except OSError:
        return "unknown"
    return "%s (vendor %s, family %s, model %s, stepping %s; %d logical CPUs on the host)" % (
        info.get("model name", "?"), info.get("vendor_id", "?"), info.get("cpu family", "?"), info.get("model", "?"),
        info.get("stepping", "?"), os.cpu_count() or 0)


def cpu_suite(threads_all):
    """The reference CPU path on the host cores for every config, one core
    (the reference is serial) and, where a sample allows, all cores."""
    return dict(
        cpu_model=cpu_model(), nproc=os.cpu_count(), threads_used=threads_all,
        config1_q8_gemv=[cpu_config1(1), cpu_config1(threads_all)],
        config3_decode_7b=cpu_config3(threads_all),
        config4_moe=[cpu_config4(1, 16, 16), cpu_config4(threads_all, 512, 64)],
        config5_mla=[cpu_config5(1), cpu_config5(threads_all)],
    )


def cpu_threads():
    """Host threads for the parallel baseline: the OpenMP setting if any (the
    GPU hosts set it to the job's CPU share), else the visible cores."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=240)
    ap.add_argument("--decode-steps", type=int, default=128)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-moe-mla", action="store_true")
    ap.add_argument("--profile-moe", type=int, default=0,
                    help="stream-launched MoE forward calls on this many tokens plus a 256 MiB copy, for counter runs")
    ap.add_argument("--profile-decode", type=int, default=0,
                    help="kernel traces and counters: this many 7B decode steps (the bench's launch mode), "
                         "the 512-token prefill, then one 256 MiB copy")
    ap.add_argument("--profile-mla", type=int, default=0,
                    help="counter runs: this many stream-launched config-5 MLA calls (8 rotating caches), "
                         "then one 256 MiB copy")
    ap.add_argument("--profile-gemv", action="store_true",
                    help="counter runs: 240 GEMV launches, then one 256 MiB device copy as the traffic calibration")
    ap.add_argument("--profile-m", type=int, default=0,
                    help="counter runs: 240 stream-launched config-2 GEMVs at this batch size")
    ap.add_argument("--profile-gemm", action="store_true",
                    help="counter runs: four M=2048 prefill GEMMs on the config-2 matrix")
    ap.add_argument("--blas-ref", action="store_true",
                    help="reference point only: the library's dense f16/bf16 GEMM (torch.matmul) on the prefill "
                         "shapes, random and all-ones operands")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (collectives are out of scope); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.blas_ref:
        print(json.dumps(blas_reference()))
        return
    dev = capi.HipComputeDevice(0)
    if args.profile_m:
        gemv_bench(dev, args.profile_m, 240, 0, graph=False)
        print(json.dumps({"profile_m": args.profile_m, "launches": 240}))
        return
    if args.profile_gemm:
        print(json.dumps(prefill_bench(dev, 2048, steps=4)))
        return
    if args.profile_moe:
        moe_bench(dev, args.profile_moe, 40, graph=False)
        a, b = dev.alloc(256 << 20, capi.U8), dev.alloc(256 << 20, capi.U8)
        capi.check(capi.lib().th_buffer_copy(b.handle, a.handle))
        dev.sync()
        print(json.dumps({"profile_moe": args.profile_moe, "calls": 40, "copy_bytes": 256 << 20}))
        return
    if args.profile_decode:
        d = decode_bench(dev, args.profile_decode)
        a, b = dev.alloc(256 << 20, capi.U8), dev.alloc(256 << 20, capi.U8)  # traffic calibration copy
        capi.check(capi.lib().th_buffer_copy(b.handle, a.handle))
        dev.sync()
        print(json.dumps({"profile_decode": args.profile_decode, "tok_s": d["tok_s"], "copy_bytes": 256 << 20}))
        return
    if args.profile_mla:
        mla_bench(dev, args.profile_mla)
        a, b = dev.alloc(256 << 20, capi.U8), dev.alloc(256 << 20, capi.U8)  # traffic calibration copy
        capi.check(capi.lib().th_buffer_copy(b.handle, a.handle))
        dev.sync()
        print(json.dumps({"profile_mla": args.profile_mla, "copy_bytes": 256 << 20}))
        return
    if args.profile_gemv:
        gemv_bench(dev, 1, 240, 0, graph="aql")  # the bench's launch mode
        a, b = dev.alloc(256 << 20, capi.U8), dev.alloc(256 << 20, capi.U8)
        capi.check(capi.lib().th_buffer_copy(b.handle, a.handle))
        dev.sync()
        print(json.dumps({"profile_gemv": True, "launches": 240, "copy_bytes": 256 << 20}))
        return
    ms = gemv_bench(dev, 1, args.steps, args.warmup)
    us = ms * 1e3 / args.steps
    gbs = GEMV_BYTES[1] / us / 1e3
    ms_stream = gemv_bench(dev, 1, args.steps, 0, graph=False)
    us_stream = ms_stream * 1e3 / args.steps
    ms_graph = gemv_bench(dev, 1, args.steps, 0, graph=True)
    us_graph = ms_graph * 1e3 / args.steps
    extra = {}
    for m in (4, 8, 16):
        msm = gemv_bench(dev, m, max(args.steps // 4, 48), 24)
        usm = msm * 1e3 / max(args.steps // 4, 48)
        extra["M=%d" % m] = dict(us=round(usm, 3), gbs=round(GEMV_BYTES[m] / usm / 1e3, 1),
                                 frac=round(GEMV_BYTES[m] / usm / 1e3 / PEAK_HBM_GBS, 4))
    q8 = q8_bench(dev, max(args.steps // 2, 100))
    prefill = [prefill_bench(dev, m) for m in (512, 2048)]
    decode = None if args.no_decode else decode_bench(dev, args.decode_steps)
    moe = None if args.no_moe_mla else [moe_bench(dev, 16, 200), moe_bench(dev, 512, 50)]
    mla = None if args.no_moe_mla else mla_bench(dev, 400)
    cpu = None if args.no_cpu else cpu_baseline()
    cpu_par = None if args.no_cpu else cpu_baseline(6.0, cpu_threads())
    cpu_all = None if args.no_cpu else cpu_suite(cpu_threads())
    out = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded xoshiro256**; int4 ~U[-8,7], f16 scales ~U[0.002,0.01], x bf16 ~N(0,1))",
        "config": {"workload": "q4 g32 GEMV 11008x4096, M=1, bf16 activations (BASELINE config 2), "
                               "%d rotating weight copies (305 MB > 256 MB MALL), launches replayed as one sequence on the "
                               "library's AQL queue (no release fences between launches; device clock stamps)"
                               % N_COPIES,
                   "timed_launches": args.steps,
                   "before_timing": "the whole timed protocol run once untimed, then: one recorded sequence: 240 untimed launches (20 passes over the copies in "
                                    "copy order), two device clock stamps back to back, one more pass, a stamp, the "
                                    "timed launches from copy 0, a last stamp; replayed once untimed, then timed. "
                                    "Time = last interval less the back-to-back stamps' span (one stamp kernel and "
                                    "its dispatch), so it covers exactly the timed launches; every timed read of a "
                                    "copy is %d launches after its previous one, and the sequence's system-scope "
                                    "fences lie outside the stamps" % N_COPIES,
                   "stream_launched": dict(us=round(us_stream, 3), gbs=round(GEMV_BYTES[1] / us_stream / 1e3, 1)),
                   "hip_graph": dict(us=round(us_graph, 3), gbs=round(GEMV_BYTES[1] / us_graph / 1e3, 1)),
                   "M_sweep": extra},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_BYTES,
                     "traffic_source": "profiles/q4_gemv_config2.md (FETCH_SIZE/WRITE_SIZE, copy-calibrated)"},
        "cpu_baseline": cpu,
        "cpu_baseline_parallel": cpu_par,
        "cpu_baselines_all_configs": cpu_all,
        "q8_config1": q8,
        "prefill_gemm_config2_matrix": prefill,
        "decode_7b": decode,
        "moe_config4": moe,
        "mla_config5": mla,
    }
    print(json.dumps(out))
    dev.close()


if __name__ == "__main__":
    main()
