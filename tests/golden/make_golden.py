"""Writes the golden fixtures under tests/golden/ by running the reference's own
CPU engine (oracle/_ref/libbrisk_ref.so, built from /root/reference/src by
oracle/Makefile) on the seeded synthetic models.  Run in the build container:

    python tests/golden/make_golden.py [names...]

Fixtures are data only: prompt ids, the greedy ids the reference picks, the
top-1 minus top-2 logit gap of each pick, and a deterministic sample of the
prompt's last-token logits (every 61st entry, the top 16, and their sum).

    python tests/golden/make_golden.py steps [names...]   # *_steps.json
    python tests/golden/make_golden.py long               # qwen3-1.7b_kv4096_steps.json

write the benchmark configs' full workloads with a sample of every step's
logits (top 8 and a strided sample); the long-context one comes from the
oracle (oracle/oracle.c), which takes a pre-filled cache.
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
    "tiny-qwen35": (12, 48),
    "tiny-qwen35w": (12, 48),
    "tiny-qwen35h": (12, 48),
    "tiny-gemma4": (12, 48),
}


def logit_sample(logits):
    top = np.argsort(-logits, kind="stable")[:16]
    return {"every61": logits[::61].tolist(), "top_idx": top.tolist(), "top_val": logits[top].tolist(),
            "sum": float(np.sum(logits.astype(np.float64)))}


# Full workloads of the benchmark configs with per-step logits: name -> (prompt length, prompt seed, greedy steps).
# Each step stores the reference's top 8 logits and a strided sample (every `stride`-th entry), so the GPU
# session's logits can be held to the tolerance at every step, not only at the prompt.
STEP_RUNS = {
    "qwen3-0.6b": (32, 7, 256),       # configs[1]
    "llama-3.2-1b": (512, 11, 128),   # configs[2]: 512-id prefill, then 128 greedy steps
    "bitnet-2b": (64, 7, 256),        # configs[4]
}
SAMPLE_POINTS = 32


def step_sample(logits, stride):
    top = np.argsort(-logits, kind="stable")[:8]
    return {"top_idx": top.tolist(), "top_val": logits[top].tolist(), "strided": logits[::stride].tolist()}


def greedy_steps(session, prompt, n_gen, stride):
    """cmd_generate's greedy loop (src/main.cpp:220-299), keeping each step's logits sample."""
    logits = session.eval(prompt)
    ids, steps = [], []
    for i in range(n_gen):
        best = int(np.argmax(logits))  # first index of the max, as Sampler::sample at temperature 0
        ids.append(best)
        steps.append(step_sample(logits, stride))
        if i + 1 < n_gen:
            logits = session.eval([best])
    return ids, steps


def steps_fixture(name):
    n_prompt, seed, n_gen = STEP_RUNS[name]
    spec = synth.SPECS[name]
    prompt = synth.prompt_ids(n_prompt, spec.vocab, seed=seed)
    stride = spec.vocab // SAMPLE_POINTS
    ref = pyoracle.Reference(synth.model_path(name), threads=os.cpu_count() or 1, max_context=n_prompt + n_gen + 8)
    t0 = time.time()
    ids, steps = greedy_steps(ref, prompt, n_gen, stride)
    ref.close()
    out = {"model": name, "seed": spec.seed, "prompt_seed": seed, "prompt": prompt.tolist(), "ids": ids, "stride": stride,
           "steps": steps, "made_by": "oracle/_ref (reference CPU engine, generic kernels)"}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"{name}_steps.json")
    with open(dst, "w") as fh:
        json.dump(out, fh)
    print(f"{name}: {n_gen} steps in {time.time() - t0:.1f}s -> {dst}", flush=True)


def long_context_fixture(n_pos=4096, n_gen=128, kv_seed=7, token=11):
    """Qwen3-1.7B-shape Q8_0 with every layer's K and V cache pre-filled to n_pos positions
    with seeded fp16 N(0,1) values (numpy default_rng(kv_seed), layer by layer, key then value), then
    greedy steps from `token`.  Run by the oracle (the C restatement, which takes a pre-filled cache)."""
    from brisk_hip import model
    name = "qwen3-1.7b"
    f, cfg, table = model.load(synth.model_path(name))
    o = pyoracle.Oracle(cfg, table, n_pos + n_gen + 8)
    rng = np.random.default_rng(kv_seed)
    for layer in range(cfg.layers):
        for value in (False, True):
            cache = o.kv(layer, value)
            cache[:, :n_pos, :] = rng.standard_normal((cfg.kv_heads, n_pos, cfg.head_dim)).astype(np.float16).view(np.uint16)
    o.set_position(n_pos)
    stride = cfg.vocab // SAMPLE_POINTS
    t0 = time.time()
    ids, steps = greedy_steps(o, [token], n_gen, stride)
    o.close()
    out = {"model": name, "seed": synth.SPECS[name].seed, "kv_positions": n_pos, "kv_seed": kv_seed, "token": token,
           "ids": ids, "stride": stride, "steps": steps,
           "made_by": "oracle/oracle.c (C restatement of the reference, pinned to oracle/_ref) on the pre-filled cache"}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), f"{name}_kv{n_pos}_steps.json")
    with open(dst, "w") as fh:
        json.dump(out, fh)
    print(f"{name} at {n_pos}: {n_gen} steps in {time.time() - t0:.1f}s -> {dst}", flush=True)


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
    args = sys.argv[1:]
    if args and args[0] == "steps":        # make_golden.py steps [names...]: the per-step fixtures
        for n in args[1:] or list(STEP_RUNS):
            steps_fixture(n)
    elif args and args[0] == "long":       # make_golden.py long: configs[3] on the pre-filled cache
        long_context_fixture()
    else:
        main(args or list(RUNS))
