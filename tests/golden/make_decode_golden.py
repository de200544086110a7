"""Writes tests/golden/llama7b_decode.json: 128 greedy decode steps of the
BASELINE config-3 model (random-init 7B shape, int4 g32 linears, f16 KV cache
prefilled to 2048 positions), computed by the CPU oracle (oracle/tang_oracle.c,
the restatement of the reference's CPU path).  Run from the repository root:
    python tests/golden/make_decode_golden.py
"""
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from llama_ref import CONFIG_7B, OracleLlama  # noqa: E402

# FIRST_TOKEN: greedy decoding from a random-init model meets near-ties (a
# top-2 logit gap comparable to the f32-vs-f64 rounding of two correct
# implementations; with first token 1 the gap at step 59 is 1.3e-5 and the
# token there depends on summation order).  Token 10 was chosen by scanning
# first tokens 1..40 on the device for trajectories that visit more than one
# token; its smallest top-2 gap in the oracle's run is 3.4e-5 (step 59) and it
# visits 3 distinct tokens.  The gaps of every step are stored with the
# tokens, and so are the five largest logits of every step, for the
# teacher-forced check.  The varied-input check is the teacher-forced golden
# of make_decode_golden_forced.py (128 distinct input tokens).
SEED, KV_SEED, PREFILL, FIRST_TOKEN, STEPS = 3, 33, 2048, 10, 128


def main():
    t0 = time.time()
    ref = OracleLlama(CONFIG_7B, SEED, KV_SEED, PREFILL)
    print("weights ready in %.1fs" % (time.time() - t0), flush=True)

    def progress(i, tok):
        print("step %d token %d (%.1fs)" % (i, tok, time.time() - t0), flush=True)

    top = []
    toks, margins, logits = ref.generate(FIRST_TOKEN, PREFILL, STEPS, progress=progress, top=top)
    out = dict(config=CONFIG_7B, seed=SEED, kv_seed=KV_SEED, prefill=PREFILL, first_token=FIRST_TOKEN, steps=STEPS,
               tokens=toks, margins=margins, last_logits_head=[float(v) for v in logits[:512]],
               top5_ids=[t[0] for t in top], top5_logits=[t[1] for t in top], logit_absmax=[t[2] for t in top],
               generator="th_synth_* (xoshiro256**), oracle or_llama_decode_step")
    with open(os.path.join(HERE, "llama7b_decode.json"), "w") as f:
        json.dump(out, f)
    print("done in %.1fs; min margin %.3e" % (time.time() - t0, min(margins)))


if __name__ == "__main__":
    main()
