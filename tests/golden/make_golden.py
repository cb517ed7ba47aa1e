"""Writes the golden fixtures under tests/golden/ by running the reference's own
CPU engine (oracle/_ref/libbrisk_ref.so, built from /root/reference/src by
oracle/Makefile) on the seeded synthetic models.  Run in the build container:

    python tests/golden/make_golden.py [names...]

Fixtures are data only: prompt ids, the greedy ids the reference picks, the
top-1 minus top-2 logit gap of each pick, and a deterministic sample of the
prompt's last-token logits (every 61st entry, the top 16, and their sum).
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "brisk-llm_amd"), os.path.join(ROOT, "oracle")]

from brisk_hip import synth  # noqa: E402
import pyoracle  # noqa: E402

# name -> (prompt length, greedy steps)
RUNS = {
    "qwen3-0.6b": (32, 256),      # configs[1]
    "bitnet-2b": (64, 64),        # configs[4] (first 64 of its 256 steps)
    "llama-3.2-1b": (64, 32),     # configs[2] shape, shorter prompt
    "tiny-qwen3": (12, 48),
    "tiny-llama": (12, 48),
    "tiny-q8": (12, 48),
    "tiny-bitnet": (12, 48),
    "tiny-q5k": (12, 48),
    "tiny-q5": (12, 48),
    "tiny-qwen2": (12, 48),
    "tiny-smollm3": (12, 48),
    "tiny-gemma3": (12, 48),
    "tiny-phi3": (12, 48),
    "tiny-llama32": (12, 48),
    "tiny-lfm2": (12, 48),
}


def logit_sample(logits):
    top = np.argsort(-logits, kind="stable")[:16]
    return {"every61": logits[::61].tolist(), "top_idx": top.tolist(), "top_val": logits[top].tolist(),
            "sum": float(np.sum(logits.astype(np.float64)))}


def main(names):
    for name in names:
        n_prompt, n_gen = RUNS[name]
        spec = synth.SPECS[name]
        path = synth.model_path(name)
        prompt = synth.prompt_ids(n_prompt, spec.vocab)
        ref = pyoracle.Reference(path, threads=os.cpu_count() or 1, max_context=n_prompt + n_gen + 8)
        t0 = time.time()
        logits = ref.eval(prompt)
        ref.rollback(0)
        ids, gaps, pre_s, gen_s = ref.generate(prompt, n_gen)
        ref.close()
        out = {"model": name, "seed": spec.seed, "prompt": prompt.tolist(), "ids": ids.tolist(),
               "gaps": [round(float(g), 6) for g in gaps], "prompt_logits": logit_sample(logits),
               "made_by": "oracle/_ref (reference CPU engine, generic kernels)"}
        dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"{name}_greedy.json")
        with open(dst, "w") as fh:
            json.dump(out, fh)
        print(f"{name}: {n_gen} ids in {time.time() - t0:.1f}s, min gap {min(gaps):.4g} -> {dst}", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or list(RUNS))
