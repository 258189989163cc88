"""The committed config-1 fixtures are reproducible from the oracle."""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def test_config1_fixture_reproduces(tmp_path):
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_config1
    import synth
    path = str(tmp_path / "tiny.st")
    synth.write_model(path, synth.TINY, seed=0)
    prompt, lg0, toks, top5, st = make_config1.compute(path)
    meta = json.load(open(os.path.join(HERE, "golden", "config1.json")))
    assert meta["prompt"] == [int(t) for t in prompt]
    assert meta["greedy"] == toks
    assert meta["top5"] == top5
    ref = np.load(os.path.join(HERE, "golden", "config1_prompt_logits.npy"))
    assert np.array_equal(lg0.astype(np.float16), ref)
    assert abs(float(np.sum(np.abs(st), dtype=np.float64)) - meta["state_abs_sum"]) < 1e-6 * meta["state_abs_sum"]
