"""Device-side helpers of the Llama parity tests; the oracle side (seeded
synthetic weights through or_llama_decode_step) is oracle/models.py."""
import ctypes

import numpy as np

from oracle.models import CONFIG_7B, CONFIG_SMALL, OracleLlama  # noqa: F401
from tang_amd import capi


def device_llama(dev, cfg, seed, kv_seed, prefill_len):
    c = capi.LlamaConfig(cfg["n_layers"], cfg["d_model"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                         cfg["d_ff"], cfg["vocab"], cfg["max_seq"], cfg["eps"], cfg["rope_theta"])
    h = ctypes.c_void_p()
    L = capi.lib()
    capi.check(L.th_llama_create(dev.handle, ctypes.byref(c), ctypes.byref(h)))
    capi.check(L.th_llama_init_synthetic(h, seed))
    capi.check(L.th_llama_fill_kv_synthetic(h, prefill_len, kv_seed))
    return h


def device_generate(model, cfg, token, pos, n_steps):
    toks = np.empty(n_steps, np.int32)
    logits = np.empty(cfg["vocab"], np.float32)
    capi.check(capi.lib().th_llama_generate(model, token, pos, n_steps, capi.ptr(toks), capi.ptr(logits)))
    return toks, logits
