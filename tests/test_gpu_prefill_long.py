"""Long prompts through the batched prefill, against the oracle.

Default path: the exact-order attention kernels (k_pre_attn_blk up to 512
positions, k_pre_attn beyond), so logits are bit-identical to the oracle's at
every prompt length, also for a prompt that continues an existing context.  Gemma 3
runs here too: its sliding layers see the last `sliding_window` positions
(src/model.cpp:1084-1088), its projections pass their post-norms, its gate is GELU.

Opt-in path (BRISK_HIP_PREFILL_ATTN=mfma): from 64 tokens on, the causal
attention runs flash style on v_mfma_f32_16x16x32_f16 with hi/lo f16 operands
(fp32 rounding of each product, not the reference's summation order).  Its
reordering can tip an int8 re-quantisation downstream, after which later layers
differ by a quantisation step: on configs[2] at 512 tokens the logits move by
about 0.03, beyond the north-star 2e-2, which is why it is not the default.  Its
tests pin what it does guarantee: on tiny models most prompts give the oracle's
logits to the bit and none moves by more than a few quantisation steps; on
configs[2] the greedy pick is the reference's and the logits stay within 0.1.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import HipSession, model, synth  # noqa: E402
import pyoracle  # noqa: E402

TOL = 2e-2
FAMILIES = ["tiny-qwen3", "tiny-llama", "tiny-q8", "tiny-bitnet", "tiny-q5k", "tiny-q5", "tiny-qwen2", "tiny-smollm3", "tiny-gemma3", "tiny-phi3", "tiny-llama32", "tiny-lfm2"]


def _session(src, ctx, mfma):
    if mfma:
        os.environ["BRISK_HIP_PREFILL_ATTN"] = "mfma"
    try:
        return HipSession(src, max_context=ctx)
    finally:
        os.environ.pop("BRISK_HIP_PREFILL_ATTN", None)


@pytest.mark.parametrize("name", FAMILIES)
@pytest.mark.parametrize("first,second", [(64, 0), (200, 0), (30, 150), (700, 0)], ids=["64", "200", "30+150", "700"])
def test_long_prompt_exact(name, first, second):
    f, cfg, table = model.load(synth.model_path(name))
    ctx = first + second + 16
    print(f"[prefill] {name}: {first} + {second} prompt ids", flush=True)
    prompt = synth.prompt_ids(first + second, cfg.vocab, seed=11)
    o = pyoracle.Oracle(cfg, table, ctx)
    want = o.eval(prompt[:first])
    if second:
        want = o.eval(prompt[first:])
    o_ids, gaps = o.generate([int(np.argmax(want))], 4)
    o.close()
    with _session((f, cfg, table), ctx, False) as s:
        got = s.eval(prompt[:first])
        if second:
            got = s.eval(prompt[first:])
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        ids = s.generate([int(np.argmax(got))], 4)
        np.testing.assert_array_equal(ids, o_ids, err_msg=f"gaps {gaps}")


# two-layer models: every extra layer re-quantises once more, so deeper stacks give fewer bit-identical prompts
@pytest.mark.parametrize("name", [n for n in FAMILIES if synth.SPECS[n].layers == 2])
def test_mfma_attention_tiny(name):
    """Eight prompts each of 64, 100 and 300 tokens: most give the oracle's logits
    bit for bit (the reordered sums round the same way after re-quantisation);
    none may move by more than a few quantisation steps."""
    f, cfg, table = model.load(synth.model_path(name))
    o = pyoracle.Oracle(cfg, table, 320)
    exact = 0
    with _session((f, cfg, table), 320, True) as s:
        for n in (64, 100, 300):
            for seed in range(1, 9):
                prompt = synth.prompt_ids(n, cfg.vocab, seed=seed)
                o.rollback(0)
                s.rollback(0)
                want, got = o.eval(prompt), s.eval(prompt)
                err = float(np.abs(got - want).max())
                exact += err == 0.0
                assert err <= 0.5, (n, seed, err)
    o.close()
    print(f"  {name}: {exact} of 24 prompts bit-identical", flush=True)
    assert exact >= 6


@pytest.mark.slow
def test_mfma_attention_llama_512():
    """configs[2] (Llama-3.2-1B-shape Q4_K_M), 512-token prompt against the
    reference engine: the default path bit for bit, the opt-in MFMA attention
    with the same greedy pick and logits within 0.1."""
    path = synth.model_path("llama-3.2-1b")
    f, cfg, table = model.load(path)
    prompt = synth.prompt_ids(512, cfg.vocab, seed=11)
    ref = pyoracle.Reference(path, threads=min(16, os.cpu_count() or 1), max_context=600)
    want = ref.eval(prompt)
    ref.close()
    for mfma in (False, True):
        with _session((f, cfg, table), 600, mfma) as s:
            got = s.eval(prompt)
        err = float(np.abs(got - want).max())
        print(f"  mfma={mfma}: max |logit diff| {err:.3g}", flush=True)
        if mfma:
            assert err <= 0.1
        else:
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        assert int(np.argmax(got)) == int(np.argmax(want))


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-q5k"])
@pytest.mark.parametrize("env", [{}, {"BRISK_HIP_PAIR_SPLIT": "1"}, {"BRISK_HIP_PREFILL_MX": "0"}, {"BRISK_HIP_PREFILL_Q4X": "1"}],
                         ids=["default", "pair-split", "packed-planes", "q4k-expanded"])
def test_prefill_gemm_variants_exact(name, env):
    """Every GEMM form of the prefill gives the oracle's logits to the bit: the fused Q4_K gate/up
    (default) and its two-launch form, the expanded-plane GEMM (default for Q6_K / Q5_K) and the
    packed-plane ones, and the expanded form for Q4_K."""
    f, cfg, table = model.load(synth.model_path(name))
    prompt = synth.prompt_ids(200, cfg.vocab, seed=5)
    o = pyoracle.Oracle(cfg, table, 216)
    want = o.eval(prompt)
    o.close()
    print(f"[prefill variants] {name} {env}", flush=True)
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        with HipSession((f, cfg, table), max_context=216) as s:
            got = s.eval(prompt)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
