"""Qwen3.5's Gated DeltaNet layers on the GPU against the oracle, bit for bit.

The recurrent layers absorb every token into a per-head state and a conv ring
(src/model.cpp:754-865), so besides the logits this pins what the reference's
rollback allows (src/model.cpp:735-752): one step back to the input state of
the last evaluated token, whichever call evaluated it (eval of many tokens,
eval_all, generate, decode), and a restart at 0 for any other earlier
position.  The device keeps the state in two halves by position parity; these
cases cross both halves many times, and a long run crosses the conv ring's
wrap-around at every position.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import BriskHipError, HipSession, model, synth  # noqa: E402
import pyoracle  # noqa: E402

NAMES = ["tiny-qwen35", "tiny-qwen35w", "tiny-qwen35h"]


def same(a, b, what):
    np.testing.assert_array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32), err_msg=what)


@pytest.fixture(scope="module", params=NAMES)
def pair(request):
    assert torch.cuda.is_available()
    name = request.param
    f, cfg, table = model.load(synth.model_path(name))
    assert cfg.arch == model.ARCH_QWEN35
    print(f"[recurrent] {name}", flush=True)
    s = HipSession((f, cfg, table), max_context=320)
    o = pyoracle.Oracle(cfg, table, 320)
    yield name, cfg, s, o
    s.close()
    o.close()


def test_step_back_after_each_kind_of_call(pair):
    name, cfg, s, o = pair
    toks = synth.prompt_ids(24, cfg.vocab, seed=9)
    for h in (s, o):
        h.rollback(0)
    first = s.eval(toks[:10])
    same(first, o.eval(toks[:10]), f"{name}: eval")
    for h in (s, o):
        h.rollback(10)  # the current position: nothing changes
        h.rollback(9)   # the last evaluated token's input state
    assert s.position == o.position == 9
    again = s.eval(toks[9:10])
    same(again, o.eval(toks[9:10]), f"{name}: eval after the step back")
    same(again, first, f"{name}: the step back re-evaluates the same token")
    # eval_all, then a step back into it
    rows = s.eval_all(toks[10:14])
    same(rows, o.eval(toks[10:14], all_logits=True), f"{name}: eval_all")
    for h in (s, o):
        h.rollback(13)
    same(s.eval(toks[13:14]), o.eval(toks[13:14]), f"{name}: eval after stepping back into eval_all")
    # generate and decode, then a step back to the last generated token's input
    ids = s.generate(toks[14:16], 6)
    o_ids, _ = o.generate(toks[14:16], 6)
    np.testing.assert_array_equal(ids, o_ids, err_msg=name)
    more = s.decode(5)
    logits = o.eval([int(o_ids[-1])])
    o_more = [int(np.argmax(logits))]
    for _ in range(4):
        logits = o.eval([o_more[-1]])
        o_more.append(int(np.argmax(logits)))
    np.testing.assert_array_equal(more, o_more, err_msg=name)
    p = s.position
    assert p == o.position
    for h in (s, o):
        h.rollback(p - 1)
    assert s.position == o.position == p - 1
    same(s.eval([int(more[-2])]), o.eval([int(o_more[-2])]), f"{name}: eval after stepping back from decode")
    # two steps back (the second finds the snapshot used), or any position but the last token's,
    # restart at 0
    for h in (s, o):
        h.rollback(p - 1)
        h.rollback(p - 2)
    assert s.position == o.position == 0
    same(s.eval(toks[:3]), o.eval(toks[:3]), f"{name}: after the restart")
    for h in (s, o):
        h.rollback(1)
    assert s.position == o.position == 0


def test_long_run_matches_the_oracle(pair):
    """300 positions: every conv ring slot and both state halves rewritten many times over."""
    name, cfg, s, o = pair
    for h in (s, o):
        h.rollback(0)
    toks = synth.prompt_ids(300, cfg.vocab, seed=11)
    same(s.eval(toks[:250]), o.eval(toks[:250]), f"{name}: 250-token eval")
    got = s.eval_all(toks[250:300])
    same(got, o.eval(toks[250:300], all_logits=True), f"{name}: 50 rows after 250 positions")


def test_set_position_is_refused(pair):
    name, cfg, s, o = pair
    with pytest.raises(BriskHipError, match="recurrent model cannot start past position 0"):
        s.set_position(5)
