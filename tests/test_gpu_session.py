"""GPU parity of the HIP session (Engine counterpart) against the oracle.

Tiny models of each family the benchmark configs use, seeded: prompt logits
within 2e-2 (fp32 accumulation-order tolerance of the north star), greedy ids
identical, eval_all rows, rollback, and the reference's error messages.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import BriskHipError, HipSession, model, synth  # noqa: E402
import pyoracle  # noqa: E402

TOL = 2e-2
FAMILIES = ["tiny-qwen3", "tiny-llama", "tiny-q8", "tiny-bitnet", "tiny-q5k", "tiny-q5", "tiny-qwen2", "tiny-smollm3", "tiny-gemma3", "tiny-phi3", "tiny-llama32", "tiny-lfm2", "tiny-qwen35", "tiny-qwen35w", "tiny-qwen35h", "tiny-gemma4"]


# the persistent token loop, one kernel per phase replayed from hipGraphs (both with the
# batched MFMA prefill for prompts), and the loop with prompts evaluated token by token
PATHS = ["loop", "graph", "tokenwise", "plain"]


@pytest.fixture(scope="module", params=[(f, p) for p in PATHS for f in FAMILIES], ids=lambda fp: f"{fp[0]}-{fp[1]}")
def pair(request):
    assert torch.cuda.is_available()
    name, path = request.param
    f, cfg, table = model.load(synth.model_path(name))
    print(f"[session] {name} ({path})", flush=True)
    env = {"tokenwise": {"BRISK_HIP_PREFILL": "0"}, "plain": {"BRISK_HIP_ATTN": "plain"}}.get(path, {"BRISK_HIP_PATH": path})
    os.environ.update(env)
    try:
        s = HipSession((f, cfg, table), max_context=256)
    finally:
        for k in env:
            del os.environ[k]
    o = pyoracle.Oracle(cfg, table, 256)
    yield name, cfg, s, o
    s.close()
    o.close()


def test_prompt_logits_and_greedy(pair):
    name, cfg, s, o = pair
    s.rollback(0)
    o.rollback(0)
    prompt = synth.prompt_ids(12, cfg.vocab)
    got, want = s.eval(prompt), o.eval(prompt)
    assert np.abs(got - want).max() <= TOL, name
    # on these contexts every path repeats the reference's arithmetic: bit for bit
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)
    assert int(np.argmax(got)) == int(np.argmax(want))
    ids = s.generate([int(np.argmax(got))], 24)
    o_ids, gaps = o.generate([int(np.argmax(want))], 24)
    np.testing.assert_array_equal(ids, o_ids, err_msg=f"{name}: gaps {gaps}")
    assert s.position == o.position == 12 + 24


def test_eval_all_and_rollback(pair):
    name, cfg, s, o = pair
    s.rollback(0)
    o.rollback(0)
    toks = synth.prompt_ids(5, cfg.vocab, seed=3)
    got, want = s.eval_all(toks), o.eval(toks, all_logits=True)
    assert got.shape == (5, cfg.vocab)
    assert np.abs(got - want).max() <= TOL
    # the batched rows (prefill GEMMs, then the output rows for all of them) are the reference's to the bit
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)
    # and decoding continues from the last row's pick
    ids = s.decode(3)
    o_ids, _ = o.generate([int(np.argmax(want[-1]))], 3)
    np.testing.assert_array_equal(ids, o_ids, err_msg=name)
    # roll back to 2 and continue: the same as evaluating from there in one go (Qwen3.5's recurrent
    # states cannot step back to 2: both restart at 0, src/model.cpp:737-750)
    s.rollback(2)
    o.rollback(2)
    assert s.position == o.position == (0 if cfg.arch == model.ARCH_QWEN35 else 2)
    g2, w2 = s.eval(toks[2:]), o.eval(toks[2:])
    assert np.abs(g2 - w2).max() <= TOL
    np.testing.assert_array_equal(g2.view(np.uint32), w2.view(np.uint32), err_msg=name)
    if cfg.arch != model.ARCH_QWEN35:
        assert np.abs(g2 - got[-1]).max() <= 1e-5
    assert s.eval_greedy([7]) == int(np.argmax(o.eval([7])))


def test_errors(pair):
    name, cfg, s, o = pair
    with pytest.raises(BriskHipError, match="token id out of range"):
        s.eval([cfg.vocab])
    with pytest.raises(BriskHipError, match="no tokens to evaluate"):
        s.eval(np.zeros(0, np.int32))
    with pytest.raises(BriskHipError, match="cannot roll forward"):
        s.rollback(s.position + 1)
    with pytest.raises(BriskHipError, match="eval_all takes 1 to 64 tokens"):
        s.eval_all(np.zeros(65, np.int32))
    s.rollback(0)
    with pytest.raises(BriskHipError, match="context length exceeded"):
        s.eval(np.zeros(257, np.int32))


def test_memory_preflight():
    """check_memory (src/memory.cpp:118-135) for HBM: a session whose estimate exceeds the free device
    memory fails before allocating, naming the shortfall; BRISK_NO_MEMORY_CHECK is the reference's override."""
    import dataclasses
    from brisk_hip.session import device_memory, estimate
    free, total = device_memory(0)
    assert 0 < free <= total
    f, cfg, table = model.load(synth.model_path("tiny-qwen3"))
    huge = dataclasses.replace(cfg, context=1 << 31)  # a 2G-token context: terabytes of cache
    need = estimate((f, huge, table), 0)
    assert need["total"] > total
    with pytest.raises(BriskHipError, match="needs about .* cache, .* of device memory is free. Try "):
        HipSession((f, huge, table), max_context=0)
    # the estimate of a real session fits, and the session works
    assert estimate((f, cfg, table), 256)["total"] < free
    with HipSession((f, cfg, table), max_context=256) as s:
        assert s.eval_greedy(synth.prompt_ids(4, cfg.vocab)) >= 0


def test_cooperative_loop_launch():
    """BRISK_HIP_COOPERATIVE=1: the token loop launched cooperatively (the runtime places the whole grid
    or refuses it) gives the same greedy ids as the oracle."""
    f, cfg, table = model.load(synth.model_path("tiny-qwen3"))
    os.environ["BRISK_HIP_COOPERATIVE"] = "1"
    try:
        s = HipSession((f, cfg, table), max_context=128)
    finally:
        del os.environ["BRISK_HIP_COOPERATIVE"]
    o = pyoracle.Oracle(cfg, table, 128)
    prompt = synth.prompt_ids(12, cfg.vocab)
    got, want = s.eval(prompt), o.eval(prompt)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    ids = s.generate([int(np.argmax(got))], 24)
    o_ids, _ = o.generate([int(np.argmax(want))], 24)
    np.testing.assert_array_equal(ids, o_ids)
    s.close()
    o.close()
