"""Oracle-side MoE layer for parity tests (test infrastructure): the same
seeded experts as th_moe_init_synthetic, run through oracle or_moe_forward."""
import ctypes

import numpy as np

import oracle
from tang_amd import capi

CONFIG4 = dict(d=2048, ff=1408, E=64, S=2, k=6)


def _q4(seed, rows, cols):
    nib, sc16 = capi.synth_q4(seed, rows, cols)
    return nib, oracle.f16_to_f32(sc16)


class OracleMoe:
    def __init__(self, cfg, seed):
        self.cfg = cfg
        d, ff, E, S = cfg["d"], cfg["ff"], cfg["E"], cfg["S"]
        self.keep = []
        self.experts = (oracle.Q4View * (3 * E))()
        self.shared = (oracle.Q4View * (3 * max(S, 1)))()
        for e in range(E + S):
            views = []
            for tid, rows, cols in ((4, ff, d), (5, ff, d), (6, d, ff)):
                nib, sc = _q4(capi.synth_seed(seed, e, tid), rows, cols)
                self.keep += [nib, sc]
                views.append(oracle.Q4View(oracle.p(nib), oracle.p(sc)))
            tgt, base = (self.experts, 3 * e) if e < E else (self.shared, 3 * (e - E))
            for i in range(3):
                tgt[base + i] = views[i]
        self.router = capi.synth_normal(capi.synth_seed(seed, 1000, 0), E * d, 0.02, capi.F32)

    def forward(self, h_bf16, T, threads=0):
        c = self.cfg
        out = np.empty(T * c["d"], np.float32)
        idx = np.empty(T * c["k"], np.int32)
        w = np.empty(T * c["k"], np.float32)
        oracle.lib().or_moe_forward(oracle.p(h_bf16), T, c["d"], c["ff"], c["E"], c["S"], c["k"],
                                    oracle.p(self.router), ctypes.cast(self.experts, ctypes.c_void_p),
                                    ctypes.cast(self.shared, ctypes.c_void_p), oracle.p(out), oracle.p(idx),
                                    oracle.p(w), threads)
        return out.reshape(T, c["d"]), idx.reshape(T, c["k"]), w.reshape(T, c["k"])


def device_moe(dev, cfg, seed):
    h = ctypes.c_void_p()
    L = capi.lib()
    capi.check(L.th_moe_create(dev.handle, cfg["d"], cfg["ff"], cfg["E"], cfg["S"], cfg["k"], ctypes.byref(h)))
    capi.check(L.th_moe_init_synthetic(h, seed))
    return h


def device_moe_forward(dev, moe, cfg, h_bf16, T):
    hb = dev.upload(h_bf16, capi.BF16)
    out = dev.alloc(T * cfg["d"])
    idx = dev.alloc(T * cfg["k"], capi.I32)
    w = dev.alloc(T * cfg["k"])
    capi.check(capi.lib().th_moe_forward(moe, hb.handle, T, out.handle, idx.handle, w.handle))
    return (out.to_numpy().reshape(T, cfg["d"]), idx.to_numpy().reshape(T, cfg["k"]),
            w.to_numpy().reshape(T, cfg["k"]))
