"""Device-side helpers of the MoE parity tests; the oracle side is
oracle/models.py (OracleMoe)."""
import ctypes

from oracle.models import CONFIG4, OracleMoe  # noqa: F401
from tang_amd import capi


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
