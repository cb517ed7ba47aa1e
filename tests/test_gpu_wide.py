"""Feed-forward rows wider than 8192 (4B-class widths: 9728 with Q6_K down rows, 14336 with Q4_0)
against the oracle, bit for bit.

The decode step's GEMVs hold their input row in LDS, up to 8192 values; a wider down projection
quantises its input to a global buffer and runs as a one-token GEMM over 256-value chunks, which
keeps the reference's block order (src/kernels.cpp:13-30 takes any width).  Such a model decodes on
the one-kernel-per-phase path; its prompts go through the batched prefill, or token by token.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import HipSession, model, synth  # noqa: E402
import pyoracle  # noqa: E402


@pytest.mark.parametrize("env", [{}, {"BRISK_HIP_PREFILL": "0"}], ids=["prefill", "tokenwise"])
@pytest.mark.parametrize("name", ["tiny-wide", "tiny-wide-q4"])
def test_wide_ffn_matches_the_oracle(name, env):
    assert torch.cuda.is_available()
    f, cfg, table = model.load(synth.model_path(name))
    assert cfg.ff > 8192
    prompt = synth.prompt_ids(24, cfg.vocab, seed=3)
    print(f"[wide] {name} ff {cfg.ff} {env}", flush=True)
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        with HipSession((f, cfg, table), max_context=64) as s:
            o = pyoracle.Oracle(cfg, table, 64)
            got, want = s.eval(prompt), o.eval(prompt)
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)
            ids = s.generate([int(np.argmax(got))], 8)
            o_ids, _ = o.generate([int(np.argmax(want))], 8)
            o.close()
        np.testing.assert_array_equal(ids, o_ids, err_msg=name)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
