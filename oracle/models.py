"""Model-level oracles (TEST INFRASTRUCTURE ONLY, like the rest of oracle/):
the seeded synthetic weights the device engines build (same generator, seeds
and tensor ids) run through the C oracle's composed functions --
or_llama_decode_step (crates/tang-train/examples/smollm.rs:215-300) and
or_moe_forward (from definition).  Used by tests/ and by bench.py's CPU
baseline leg only.
"""
import concurrent.futures
import ctypes

import numpy as np

import oracle
from tang_amd import capi

T_WQ, T_WK, T_WV, T_WO, T_WG, T_WU, T_WD, T_ATTN_NORM, T_FFN_NORM = range(9)
T_EMBED, T_FINAL_NORM, T_LM_HEAD = 10, 11, 12
T_KCACHE, T_VCACHE = 20, 21
NORM_STD = 0.02

CONFIG_7B = dict(n_layers=32, d_model=4096, n_heads=32, n_kv_heads=32, head_dim=128, d_ff=11008, vocab=32000,
                 max_seq=2176, eps=1e-5, rope_theta=1e4)
CONFIG_SMALL = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, d_ff=512, vocab=1000,
                    max_seq=192, eps=1e-5, rope_theta=1e4)


def _q4(seed, rows, cols):
    nib, sc16 = capi.synth_q4(seed, rows, cols)
    return nib, oracle.f16_to_f32(sc16)


def _q4_from_f32(w, rows, cols):
    """quantize_matrix_q4 (quantize.rs:208-221), block scales rounded to f16
    as the engine stores them."""
    blocks = oracle.quantize_matrix_q4(np.ascontiguousarray(w, np.float32).reshape(-1), rows, cols)
    nib = np.ascontiguousarray(blocks["values"]).reshape(-1)
    return nib, oracle.f16_to_f32(oracle.f32_to_f16(blocks["scale"]))


LINEAR_NAMES = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj",
                "wo": "self_attn.o_proj", "wg": "mlp.gate_proj", "wu": "mlp.up_proj", "wd": "mlp.down_proj"}


class OracleLlama:
    """Seeded synthetic weights (as th_llama_init_synthetic), or with
    `tensors` (Llama tensor name -> f32 array) the weights a safetensors
    file gives th_llama_load_safetensors.  `workers` threads generate the
    tensors (the result does not depend on it)."""

    def __init__(self, cfg, seed, kv_seed, prefill_len, tensors=None, workers=1):
        self.cfg = cfg
        c = cfg
        L, d, ff = c["n_layers"], c["d_model"], c["d_ff"]
        qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
        self.keep = []
        views = {k: (oracle.Q4View * L)() for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
        shapes = {"wq": (T_WQ, qd, d), "wk": (T_WK, kvd, d), "wv": (T_WV, kvd, d), "wo": (T_WO, d, d),
                  "wg": (T_WG, ff, d), "wu": (T_WU, ff, d), "wd": (T_WD, d, ff)}
        # the seeded tensors are independent: generated in a thread pool (the
        # generator is C code called through ctypes, which releases the GIL)
        jobs = [(l, name) for l in range(L) for name in shapes]

        def make(job):
            l, name = job
            tid, rows, cols = shapes[name]
            if tensors is None:
                return _q4(capi.synth_seed(seed, l, tid), rows, cols)
            return _q4_from_f32(tensors["model.layers.%d.%s.weight" % (l, LINEAR_NAMES[name])], rows, cols)

        with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
            made = list(ex.map(make, jobs))
        for (l, name), (nib, sc) in zip(jobs, made):
            self.keep += [nib, sc]
            views[name][l] = oracle.Q4View(oracle.p(nib), oracle.p(sc))
        del made
        if tensors is None:
            lm_nib, lm_sc = _q4(capi.synth_seed(seed, L, T_LM_HEAD), c["vocab"], d)
            self.embed = capi.synth_normal(capi.synth_seed(seed, L, T_EMBED), c["vocab"] * d, NORM_STD, capi.BF16)
            self.attn_norm = np.concatenate([capi.synth_normal(capi.synth_seed(seed, l, T_ATTN_NORM), d, NORM_STD,
                                                               capi.BF16) for l in range(L)])
            self.ffn_norm = np.concatenate([capi.synth_normal(capi.synth_seed(seed, l, T_FFN_NORM), d, NORM_STD,
                                                              capi.BF16) for l in range(L)])
            self.final_norm = capi.synth_normal(capi.synth_seed(seed, L, T_FINAL_NORM), d, NORM_STD, capi.BF16)
        else:
            emb = tensors["model.embed_tokens.weight"]
            lm_nib, lm_sc = _q4_from_f32(tensors.get("lm_head.weight", emb), c["vocab"], d)
            self.embed = oracle.f32_to_bf16(emb.reshape(-1))
            self.attn_norm = np.concatenate([oracle.f32_to_bf16(tensors["model.layers.%d.input_layernorm.weight" % l])
                                             for l in range(L)])
            self.ffn_norm = np.concatenate([oracle.f32_to_bf16(
                tensors["model.layers.%d.post_attention_layernorm.weight" % l]) for l in range(L)])
            self.final_norm = oracle.f32_to_bf16(tensors["model.norm.weight"])
        self.keep += [lm_nib, lm_sc]
        self.cos, self.sin = oracle.rope_tables(c["head_dim"], c["max_seq"], c["rope_theta"])
        self.kc = np.zeros((L, c["max_seq"], kvd), np.uint16)
        self.vc = np.zeros((L, c["max_seq"], kvd), np.uint16)
        def fill(l):
            n = prefill_len * kvd
            self.kc[l, :prefill_len] = capi.synth_normal(capi.synth_seed(kv_seed, l, T_KCACHE), n, 1.0,
                                                         capi.F16).reshape(prefill_len, kvd)
            self.vc[l, :prefill_len] = capi.synth_normal(capi.synth_seed(kv_seed, l, T_VCACHE), n, 1.0,
                                                         capi.F16).reshape(prefill_len, kvd)

        with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
            list(ex.map(fill, range(L)))
        self.W = oracle.LlamaWeights(
            oracle.p(self.embed), oracle.p(self.attn_norm), oracle.p(self.ffn_norm), oracle.p(self.final_norm),
            ctypes.cast(views["wq"], ctypes.c_void_p), ctypes.cast(views["wk"], ctypes.c_void_p),
            ctypes.cast(views["wv"], ctypes.c_void_p), ctypes.cast(views["wo"], ctypes.c_void_p),
            ctypes.cast(views["wg"], ctypes.c_void_p), ctypes.cast(views["wu"], ctypes.c_void_p),
            ctypes.cast(views["wd"], ctypes.c_void_p), oracle.Q4View(oracle.p(lm_nib), oracle.p(lm_sc)),
            oracle.p(self.cos), oracle.p(self.sin))
        self.views = views
        self.ccfg = oracle.LlamaCfg(c["n_layers"], d, c["n_heads"], c["n_kv_heads"], c["head_dim"], ff, c["vocab"],
                                    c["max_seq"], c["eps"])

    def step(self, token, pos, threads=0):
        logits = np.empty(self.cfg["vocab"], np.float32)
        tok = oracle.lib().or_llama_decode_step(ctypes.byref(self.ccfg), ctypes.byref(self.W), oracle.p(self.kc),
                                                oracle.p(self.vc), int(token), int(pos), oracle.p(logits), threads)
        return tok, logits

    def generate(self, token, pos, n_steps, threads=0, progress=None, top=None):
        """Greedy steps; with a list `top`, appends each step's five largest
        logits as (ids, values, max |logit|)."""
        toks, margins = [], []
        logits = None
        for i in range(n_steps):
            token, logits = self.step(token, pos + i, threads)
            top2 = np.sort(logits)[-2:]
            toks.append(int(token))
            margins.append(float(top2[1] - top2[0]))
            if top is not None:
                ids = np.argsort(-logits, kind="stable")[:5]
                top.append(([int(j) for j in ids], [float(logits[j]) for j in ids], float(np.abs(logits).max())))
            if progress:
                progress(i, token)
        return toks, margins, logits




CONFIG4 = dict(d=2048, ff=1408, E=64, S=2, k=6)


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


