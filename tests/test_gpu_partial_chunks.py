"""Rows of 32-value blocks that end inside a 256-value chunk, through the batched prefill, against
the oracle bit for bit.

The prefill's GEMMs stage their rows in 256-value chunks; a Q4_0 / Q8_0 row of 1152 values
(Gemma-3-1B) ends inside its fifth.  The last chunk then reads and adds only the row's blocks
(src/quant.cpp:445-482, each block's term in order), so the prompt's logits, every row of
eval_all, and the greedy steps after it equal the oracle's.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import HipSession, model, synth  # noqa: E402
import pyoracle  # noqa: E402


@pytest.mark.parametrize("name", ["tiny-gemma3w", "tiny-q8w"])
def test_partial_chunk_prefill_matches_the_oracle(name):
    assert torch.cuda.is_available()
    f, cfg, table = model.load(synth.model_path(name))
    assert cfg.embd % 256 != 0 and cfg.ff % 256 != 0
    prompt = synth.prompt_ids(40, cfg.vocab, seed=21)
    print(f"[partial chunks] {name} embd {cfg.embd} ff {cfg.ff}", flush=True)
    with HipSession((f, cfg, table), max_context=96) as s:
        o = pyoracle.Oracle(cfg, table, 96)
        got, want = s.eval(prompt), o.eval(prompt)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)
        ids = s.generate([int(np.argmax(got))], 6)
        o_ids, _ = o.generate([int(np.argmax(want))], 6)
        np.testing.assert_array_equal(ids, o_ids, err_msg=name)
        for h in (s, o):
            h.rollback(0)
        rows = s.eval_all(prompt[:20])
        np.testing.assert_array_equal(rows.view(np.uint32), o.eval(prompt[:20], all_logits=True).view(np.uint32), err_msg=name)
        o.close()
