"""Writes the config-1 golden fixtures from the CPU oracle.

Config 1: tiny RWKV-7 (12 layers, d_model 768,
12 heads x 64, FFN 3072, vocab 65536, LoRA 64/64/32/128), random-init with
seed 0, fp32 N(0, 0.02^2); a 64-token uniform random prompt (PCG64 seeded
with (0, 1)), then 32 greedy tokens.

Outputs (beside this script):
  config1.json               prompt ids, greedy ids, per-step top-5 ids,
                             final-state checksums
  config1_prompt_logits.npy  logits after the prompt (float16 to stay small)

Run: python tests/golden/make_config1.py   (about a minute on one core)
"""
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "rwkv-rsv_amd"), os.path.join(ROOT, "oracle")]

import synth  # noqa: E402
import oracle  # noqa: E402


def compute(path):
    m = oracle.Model(path)
    prompt = synth.prompt(synth.TINY, 64, seed=0)
    st = m.init_state()
    lg0 = m.forward(prompt, st)
    toks, top5 = [], []
    lg = lg0
    for _ in range(32):
        t = oracle.argmax(lg)
        toks.append(t)
        top5.append([int(i) for i in np.argsort(-lg, kind="stable")[:5]])
        lg = m.forward([t], st)
    return prompt, lg0, toks, top5, st


def main():
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.st")
        synth.write_model(path, synth.TINY, seed=0)
        prompt, lg0, toks, top5, st = compute(path)
    meta = {
        "config": "BASELINE configs[0]: tiny RWKV-7 seed 0, 64-token prompt + 32 greedy",
        "prompt": [int(t) for t in prompt],
        "greedy": [int(t) for t in toks],
        "top5": top5,
        "state_len": int(st.size),
        "state_sum": float(np.sum(st, dtype=np.float64)),
        "state_abs_sum": float(np.sum(np.abs(st), dtype=np.float64)),
    }
    with open(os.path.join(HERE, "config1.json"), "w") as f:
        json.dump(meta, f, indent=1)
    np.save(os.path.join(HERE, "config1_prompt_logits.npy"), lg0.astype(np.float16))
    print("greedy:", toks)


if __name__ == "__main__":
    main()
