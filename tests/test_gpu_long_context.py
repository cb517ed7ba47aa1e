"""Long contexts: KV caches pre-filled with seeded fp16 N(0,1) values (as configs[3]
does to 4096 positions), then decode, against the oracle running on the same
pre-filled cache (brisk_hip_session_kv_cache / set_position on the GPU,
or_session_kv / set_position in the oracle).

Every attention path keeps the reference's order at every length
(src/kernels_f32.cpp:256-284): the token loop's spread and resident attentions,
its pooled exact attention, and the one-kernel-per-phase path's exact attention,
whose scores go to global memory past the LDS limit.  A session whose context no
loop attention takes whole (more than 4 query heads a kv head, partial rotary,
or heads-per-kv x length beyond the spread attention's 16384 scores, as
Llama-3.2-1B beyond 4096 positions) runs on the one-kernel-per-phase path.  So
the tiny models' logits are bit-identical to the oracle's, and the full-size
case is held step by step to the north-star tolerance (max-abs 2e-2) with
identical greedy ids.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import HipSession, model, synth  # noqa: E402
import pyoracle  # noqa: E402

TOL = 2e-2


def prefill_kv(s, o, cfg, n_pos, seed):
    """Seeded fp16 N(0,1) keys and values for positions [0, n_pos) of every layer, into both sessions."""
    rng = np.random.default_rng(seed)
    for layer in range(cfg.layers):
        for value in (False, True):
            cache = o.kv(layer, value)  # [kv_heads][max_context][head_dim], oracle-owned host memory
            vals = rng.standard_normal((cfg.kv_heads, n_pos, cfg.head_dim)).astype(np.float16)
            cache[:, :n_pos, :] = vals.view(np.uint16)
            ptr, nbytes = s.kv_cache(layer, value)
            assert cache.nbytes == nbytes
            _h2d(ptr, np.ascontiguousarray(cache), nbytes)
    s.set_position(n_pos)
    o.set_position(n_pos)


def _h2d(dst_ptr, host, nbytes):
    """Host-to-device copy into a raw device pointer (the session's cache)."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    assert hip.hipMemcpy(C.c_void_p(dst_ptr), C.c_void_p(host.ctypes.data), nbytes, 1) == 0  # hipMemcpyHostToDevice


# tiny-gemma3: its sliding layers see only the last 8 of the 900 positions, its global layer all of them
@pytest.mark.parametrize("name,n_pos,steps", [("tiny-qwen3", 900, 6), ("tiny-llama", 700, 6), ("tiny-gemma3", 900, 6),
                                                 ("tiny-phi3", 900, 6)])
def test_long_attention_tiny(name, n_pos, steps):
    f, cfg, table = model.load(synth.model_path(name))
    print(f"[long] {name}: KV pre-filled to {n_pos}", flush=True)
    with HipSession((f, cfg, table), max_context=n_pos + 16) as s:
        o = pyoracle.Oracle(cfg, table, n_pos + 16)
        prefill_kv(s, o, cfg, n_pos, seed=5)
        tok = [17]
        got, want = s.eval(tok), o.eval(tok)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))  # the reference's order: the same bits
        ids = s.generate([int(np.argmax(got))], steps)
        o_ids, gaps = o.generate([int(np.argmax(want))], steps)
        np.testing.assert_array_equal(ids, o_ids, err_msg=f"gaps {gaps}")
        o.close()


@pytest.mark.parametrize("n_pos", [300, 9000])
def test_long_plain_attention(n_pos):
    """The plain attention (BRISK_HIP_ATTN=plain) at 300 positions (weights in LDS) and at 9000 (past its
    8192-position LDS window: the weights recomputed per position), bit-identical to the oracle."""
    import os
    f, cfg, table = model.load(synth.model_path("tiny-qwen3-long"))
    print(f"[long] tiny-qwen3-long plain attention: KV pre-filled to {n_pos}", flush=True)
    os.environ["BRISK_HIP_ATTN"] = "plain"
    try:
        s = HipSession((f, cfg, table), max_context=n_pos + 16)
    finally:
        del os.environ["BRISK_HIP_ATTN"]
    with s:
        o = pyoracle.Oracle(cfg, table, n_pos + 16)
        prefill_kv(s, o, cfg, n_pos, seed=9)
        got, want = s.eval([23]), o.eval([23])
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        ids = s.generate([int(np.argmax(got))], 4)
        o_ids, gaps = o.generate([int(np.argmax(want))], 4)
        np.testing.assert_array_equal(ids, o_ids, err_msg=f"gaps {gaps}")
        o.close()


@pytest.mark.slow
def test_qwen3_1_7b_at_4096():
    """configs[3] at full size: Qwen3-1.7B-shape Q8_0, 4096 pre-filled positions, then decode."""
    f, cfg, table = model.load(synth.model_path("qwen3-1.7b"))
    n_pos = 4096
    print(f"[long] qwen3-1.7b: KV pre-filled to {n_pos}", flush=True)
    with HipSession((f, cfg, table), max_context=n_pos + 8) as s:
        o = pyoracle.Oracle(cfg, table, n_pos + 8)
        prefill_kv(s, o, cfg, n_pos, seed=7)
        got, want = s.eval([11]), o.eval([11])
        print(f"  max |logit diff| {np.abs(got - want).max():.3g}", flush=True)
        assert np.abs(got - want).max() <= TOL
        ids = s.generate([int(np.argmax(got))], 2)
        o_ids, gaps = o.generate([int(np.argmax(want))], 2)
        np.testing.assert_array_equal(ids, o_ids, err_msg=f"gaps {gaps}")
        o.close()


def test_llama_1b_beyond_the_spread_attention():
    """Llama-3.2-1B shape (4 query heads a kv head): 4200 pre-filled positions, past the loop's
    attentions (4 x 4200 scores), so the session decodes on the one-kernel-per-phase path with
    its global-memory exact attention.  32 greedy steps; at every step the oracle evaluates the
    same token on its own cache and the logits agree within 2e-2."""
    f, cfg, table = model.load(synth.model_path("llama-3.2-1b"))
    n_pos, steps = 4200, 32
    print(f"[long] llama-3.2-1b: KV pre-filled to {n_pos}, {steps} teacher-forced steps", flush=True)
    with HipSession((f, cfg, table), max_context=n_pos + steps + 8) as s:
        o = pyoracle.Oracle(cfg, table, n_pos + steps + 8)
        prefill_kv(s, o, cfg, n_pos, seed=11)
        tok, worst, exact = 23, 0.0, 0
        for step in range(steps):
            got, want = s.eval([tok]), o.eval([tok])
            diff = float(np.abs(got - want).max())
            worst = max(worst, diff)
            exact += int(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
            assert diff <= TOL, f"step {step}: max |logit diff| {diff}"
            assert int(np.argmax(got)) == int(np.argmax(want)), f"step {step}: greedy ids differ"
            tok = int(np.argmax(got))
        print(f"  worst per-step logit diff {worst:.3g}; {exact} of {steps} steps bit-identical", flush=True)
        o.close()
