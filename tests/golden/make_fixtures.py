#!/usr/bin/env python3
"""Write the golden fixtures of the synthetic workloads with the oracle.

tiny_f32.json: the tiny F32 model (seed 42), prompt [3,1,4,1,5,9,2,6]: the
last-position logits and 24 greedy tokens after the prompt.
gqa_q8.json: the GQA Q8_0 model (seed 43), its 16-token random prompt, the
last-position logits' argmax and 32 greedy tokens after it.

The reference's own fixtures (tests/fixtures/tiny_logits.json,
tiny32_logits.json) were captured on model files that its repository does
not ship, so they cannot be replayed here; these fixtures pin the oracle
against drift and give the GPU path a stored target.

Usage: python tests/golden/make_fixtures.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import talos_amd as T  # noqa: E402
from oracle import oracle as O  # noqa: E402
from talos_amd import configs  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def greedy(model, prompt, n):
    for p, t in enumerate(prompt):
        lg = model.forward(t, p)
    last = lg.copy()
    toks = []
    tok = O.argmax(lg)
    for i in range(n):
        toks.append(int(tok))
        lg = model.forward(tok, len(prompt) + i)
        tok = O.argmax(lg)
    return last, toks


def main():
    wl = configs.tiny_f32()
    m = O.OracleModel(T.synth_bytes(wl.spec, nthreads=4), nthreads=4)
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    last, toks = greedy(m, prompt, 24)
    m.close()
    with open(os.path.join(HERE, "tiny_f32.json"), "w") as f:
        json.dump({"workload": "tiny_f32", "seed": wl.spec.seed, "prompt": prompt,
                   "last_logits": [float(np.float32(v)) for v in last], "greedy": toks}, f)

    wl = configs.gqa_q8()
    m = O.OracleModel(T.synth_bytes(wl.spec, nthreads=4), nthreads=4)
    prompt = [int(x) for x in np.random.default_rng(wl.spec.seed + 1).integers(0, wl.spec.vocab_size,
                                                                                wl.prompt_len)]
    last, toks = greedy(m, prompt, 32)
    m.close()
    with open(os.path.join(HERE, "gqa_q8.json"), "w") as f:
        json.dump({"workload": "gqa_q8", "seed": wl.spec.seed, "prompt": prompt,
                   "last_argmax": int(O.argmax(last)), "last_logits_head": [float(v) for v in last[:64]],
                   "greedy": toks}, f)


if __name__ == "__main__":
    main()
