"""The graph-path families at full size against the oracle, bit for bit.

bench.py times these shapes (brisk_hip/synth.py: Gemma-3-1B, LFM2-1.2B, a Qwen3.5 shape and a
Gemma 4 shape, synthetic weights).  Here each one's prompt logits and first greedy steps must
equal the oracle's, which is pinned bitwise against the reference's engine on the tiny shapes
of the same families.  At these sizes the oracle runs a few seconds a token, so the runs are
short: a 5-id prompt and 3 greedy steps.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import HipSession, model, synth  # noqa: E402
import pyoracle  # noqa: E402


@pytest.mark.parametrize("name", ["gemma3-1b", "lfm2-1.2b", "qwen35-0.8b", "gemma4-e2b"])
def test_full_size_family_matches_the_oracle(name):
    assert torch.cuda.is_available()
    print(f"[family] {name}", flush=True)
    f, cfg, table = model.load(synth.model_path(name))
    prompt = synth.prompt_ids(5, cfg.vocab, seed=13)
    with HipSession((f, cfg, table), max_context=64) as s:
        o = pyoracle.Oracle(cfg, table, 64)
        got, want = s.eval(prompt), o.eval(prompt)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)
        ids = s.generate([int(np.argmax(got))], 3)
        o_ids, _ = o.generate([int(np.argmax(want))], 3)
        o.close()
    np.testing.assert_array_equal(ids, o_ids, err_msg=name)
