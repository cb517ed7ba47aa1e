"""The drop-in binding on the GPU: brisk-llm_amd/binding/hip_session.h (class HipSession : Engine),
made from the reference's own Model(file, repack = false) and driven the way the reference's code
drives an Engine (oracle/hip_engine_shim.cpp, built into oracle/_ref/libhip_engine.so):

  - cmd_generate's greedy loop over Engine::eval (src/main.cpp:287-299) and the on-device
    generate_greedy fast path: configs[1]'s 256 ids equal the reference Session's (the golden
    fixture), and every family's tiny model gives the reference's ids and prompt logits;
  - cmd_generate --draft (src/main.cpp:236-276): the reference's Speculator over the HipSession
    target, with the lookup drafter and with a CPU ModelDrafter, settles exactly the greedy ids;
  - serve --gpu (src/server.cpp:237-265, :380-395): the warm-up pass, then turns that reuse the
    common prefix of the cache, whose logits equal a fresh evaluation of the whole conversation;
  - Engine::log_likelihood (src/engine.cpp:10-33, the perplexity command) over eval_all.
"""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import model, synth  # noqa: E402
import pyoracle  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
TOL = 2e-2
FAMILIES = ["tiny-qwen3", "tiny-llama", "tiny-q8", "tiny-bitnet", "tiny-q5k", "tiny-q5", "tiny-qwen2", "tiny-smollm3",
            "tiny-gemma3", "tiny-phi3", "tiny-llama32", "tiny-lfm2", "tiny-qwen35", "tiny-qwen35w", "tiny-qwen35h", "tiny-gemma4"]


@pytest.fixture(scope="module", autouse=True)
def needs_library():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert pyoracle.hip_engine_available(), "oracle/_ref/libhip_engine.so is not built"


def test_configs1_greedy_through_the_engine_interface():
    with open(os.path.join(HERE, "golden", "qwen3-0.6b_greedy.json")) as fh:
        g = json.load(fh)
    prompt, want = np.array(g["prompt"], np.int32), np.array(g["ids"], np.int32)
    print(f"[binding] qwen3-0.6b: {len(want)} greedy ids through HipSession : Engine", flush=True)
    e = pyoracle.HipEngine(synth.model_path("qwen3-0.6b"), len(prompt) + len(want) + 8, synth.SPECS["qwen3-0.6b"].vocab)
    ids = e.generate(prompt, len(want))
    np.testing.assert_array_equal(ids, want)
    e.rollback(0)
    ids = e.generate(prompt, len(want), on_device=True)
    np.testing.assert_array_equal(ids, want)
    assert e.position == len(prompt) + len(want) - 1
    e.close()


@pytest.mark.parametrize("name", FAMILIES)
def test_families_through_the_engine_interface(name):
    path = synth.model_path(name)
    vocab = synth.SPECS[name].vocab
    prompt = synth.prompt_ids(12, vocab)
    print(f"[binding] {name}", flush=True)
    ref = pyoracle.Reference(path, threads=4, max_context=128)
    want = ref.eval(prompt)
    ref.rollback(0)
    want_ids, _, _, _ = ref.generate(prompt, 24)
    ref.close()
    e = pyoracle.HipEngine(path, 128, vocab)
    got = e.eval(prompt)
    assert np.abs(got - want).max() <= TOL
    e.rollback(0)
    np.testing.assert_array_equal(e.generate(prompt, 24), want_ids)
    e.close()


@pytest.mark.parametrize("drafter", ["lookup", "model"])
def test_speculative_decoding_settles_the_greedy_ids(drafter):
    name = "tiny-qwen3"
    path = synth.model_path(name)
    vocab = synth.SPECS[name].vocab
    prompt = synth.prompt_ids(12, vocab)
    ref = pyoracle.Reference(path, threads=4, max_context=256)
    want, _, _, _ = ref.generate(prompt, 64)
    ref.close()
    e = pyoracle.HipEngine(path, 256, vocab)
    ids, stats = e.speculative(prompt, 64, draft_tokens=8, draft_path=path if drafter == "model" else None, threads=4)
    print(f"[binding] speculative ({drafter} drafter): {stats}", flush=True)
    np.testing.assert_array_equal(ids, want)
    if drafter == "model":  # the same model drafting: every guess is right, so eval_all verifies whole batches
        assert stats["accepted"] > 0 and stats["rounds"] > 0
    e.close()


def test_serve_turns_reuse_the_common_prefix():
    name = "tiny-llama"
    path = synth.model_path(name)
    vocab = synth.SPECS[name].vocab
    a = synth.prompt_ids(20, vocab, seed=3)
    b = synth.prompt_ids(9, vocab, seed=4)
    e = pyoracle.HipEngine(path, 256, vocab)
    e.serve_warmup(1)
    assert e.position == 0
    l1, reused1 = e.serve_prefill(a)
    assert reused1 == 0
    reply = list(np.argsort(-l1)[:5].astype(np.int32))  # five reply tokens the server would have streamed
    e.serve_extend(reply)
    turn2 = np.concatenate([a, reply, b]).astype(np.int32)
    l2, reused2 = e.serve_prefill(turn2)
    assert reused2 == len(a) + len(reply)
    # the same conversation evaluated from scratch, on a fresh engine and on the reference
    f = pyoracle.HipEngine(path, 256, vocab)
    fresh = f.eval(turn2)
    f.close()
    np.testing.assert_array_equal(l2.view(np.uint32), fresh.view(np.uint32))
    ref = pyoracle.Reference(path, threads=4, max_context=256)
    assert np.abs(l2 - ref.eval(turn2)).max() <= TOL
    ref.close()
    # a turn that is a prefix of the cache re-evaluates only its last token
    l3, reused3 = e.serve_prefill(turn2[:10])
    assert reused3 == 9
    e.close()


def test_log_likelihood_matches_the_reference():
    name = "tiny-qwen3"
    path = synth.model_path(name)
    vocab = synth.SPECS[name].vocab
    text = synth.prompt_ids(100, vocab, seed=9)  # two eval_all chunks of at most 64 tokens
    ref = pyoracle.Reference(path, threads=4, max_context=256)
    want = ref.log_likelihood(text)
    ref.close()
    e = pyoracle.HipEngine(path, 256, vocab)
    got = e.log_likelihood(text)
    e.close()
    print(f"[binding] log-likelihood {got:.6f} (reference {want:.6f})", flush=True)
    assert abs(got - want) <= 1e-6 * abs(want) + 1e-6
