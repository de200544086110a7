"""Writes tests/golden/llama7b_forced.json: 128 teacher-forced decode steps
of the BASELINE config-3 model (random-init 7B shape, int4 g32 linears, f16
KV cache prefilled to 2048 positions) on 128 distinct seeded input tokens,
computed by the CPU oracle (oracle/tang_oracle.c, the restatement of the
reference's CPU path).  Step i feeds token tokens_in[i] at position 2048+i;
the K/V rows each step appends are its own input's, so every step reads a
different embedding row and a different attention history.  Stored per step:
the greedy token, the top-2 gap, the five largest logits with their ids,
max |logit| and the first 256 logits.  Run from the repository root:
    python tests/golden/make_decode_golden_forced.py
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from llama_ref import CONFIG_7B, OracleLlama  # noqa: E402

SEED, KV_SEED, PREFILL, STEPS, TOKEN_SEED, HEAD = 3, 33, 2048, 128, 2026, 256


def main():
    t0 = time.time()
    toks_in = [int(t) for t in np.random.default_rng(TOKEN_SEED).choice(CONFIG_7B["vocab"], STEPS, replace=False)]
    ref = OracleLlama(CONFIG_7B, SEED, KV_SEED, PREFILL)
    print("weights ready in %.1fs" % (time.time() - t0), flush=True)
    out_tok, margins, top_ids, top_vals, absmax, heads = [], [], [], [], [], []
    for i, t in enumerate(toks_in):
        tok, logits = ref.step(t, PREFILL + i)
        order = np.argsort(-logits, kind="stable")
        top2 = logits[order[:2]]
        out_tok.append(int(tok))
        margins.append(float(top2[0] - top2[1]))
        top_ids.append([int(j) for j in order[:5]])
        top_vals.append([float(logits[j]) for j in order[:5]])
        absmax.append(float(np.abs(logits).max()))
        heads.append([float(v) for v in logits[:HEAD]])
        print("step %d in %d out %d (%.1fs)" % (i, t, tok, time.time() - t0), flush=True)
    out = dict(config=CONFIG_7B, seed=SEED, kv_seed=KV_SEED, prefill=PREFILL, steps=STEPS, token_seed=TOKEN_SEED,
               tokens_in=toks_in, tokens=out_tok, margins=margins, top5_ids=top_ids, top5_logits=top_vals,
               logit_absmax=absmax, logits_head=heads,
               generator="th_synth_* (xoshiro256**), oracle or_llama_decode_step, teacher-forced")
    with open(os.path.join(HERE, "llama7b_forced.json"), "w") as f:
        json.dump(out, f)
    print("done in %.1fs; min margin %.3e; distinct outputs %d" % (time.time() - t0, min(margins), len(set(out_tok))))


if __name__ == "__main__":
    main()
