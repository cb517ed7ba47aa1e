"""Full-size (and tiny) models against the reference's own greedy runs.

tests/golden/*_greedy.json were written by tests/golden/make_golden.py from the
reference's CPU engine (oracle/_ref) on the same seeded GGUF files.  The HIP
session must pick the same greedy ids and reproduce the sampled prompt logits
(within the 2e-2 tolerance; in practice bit for bit on these contexts).
"""
import glob
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import HipSession, synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*_greedy.json")))


@pytest.mark.parametrize("fixture", FIXTURES, ids=[os.path.basename(f).replace("_greedy.json", "") for f in FIXTURES])
def test_greedy_matches_reference(fixture):
    with open(fixture) as fh:
        g = json.load(fh)
    print(f"[model] {g['model']}: {len(g['prompt'])} prompt ids, {len(g['ids'])} greedy", flush=True)
    path = synth.model_path(g["model"])
    prompt = np.array(g["prompt"], np.int32)
    with HipSession(path, max_context=len(prompt) + len(g["ids"]) + 8) as s:
        logits = s.eval(prompt)
        pl = g["prompt_logits"]
        np.testing.assert_allclose(logits[::61], np.array(pl["every61"], np.float32), rtol=0, atol=2e-2)
        np.testing.assert_allclose(logits[pl["top_idx"]], np.array(pl["top_val"], np.float32), rtol=0, atol=2e-2)
        exact = np.array_equal(logits[::61], np.array(pl["every61"], np.float32))
        print(f"  prompt logits bit-identical on the sample: {exact}", flush=True)
        first = int(np.argmax(logits))
        ids = np.concatenate([[first], s.decode(len(g["ids"]) - 1)])
    want = np.array(g["ids"], np.int32)
    mism = np.flatnonzero(ids != want)
    assert len(mism) == 0, f"first divergence at step {mism[0]} (reference gap there {g['gaps'][mism[0]]})"
