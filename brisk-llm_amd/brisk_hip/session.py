"""HipSession: the Engine interface (src/engine.h:13-37) over the C ABI.

Mirrors the reference's ``Session`` / ``MetalSession``: ``eval`` returns the
last token's logits, ``eval_all`` every token's (1..64 tokens), ``rollback``
forgets from a position on, ``position`` is the sequence length so far, and
``log_likelihood`` is ``Engine::log_likelihood`` (src/engine.cpp:10-33).
Errors raise ``BriskHipError`` (a RuntimeError) with the reference's messages.
"""
from __future__ import annotations

import atexit
import ctypes as C
import weakref

import numpy as np

from . import lib as _lib
from . import model as _model


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _c_args(c, table):
    """The C ABI's config and tensor table for a ModelConfig and tensor list (plus what keeps them alive)."""
    hc = _lib.HipConfig(c.arch, c.vocab, c.embd, c.layers, c.heads, c.kv_heads, c.head_dim, c.ff, c.context,
                        c.rope_base, c.eps, c.sliding_window, c.rope_base_local, c.rope_scale, c.final_softcap,
                        c.rope_dim, c.rope_attn_factor, c.rope_original_context, c.conv_taps)
    hc.ssm_state, hc.ssm_k_heads, hc.ssm_v_heads = c.ssm_state, c.ssm_k_heads, c.ssm_v_heads
    hc.ssm_inner, hc.ssm_conv = c.ssm_inner, c.ssm_conv
    hc.head_dim_local, hc.kv_from_start, hc.ple_dim = c.head_dim_local, c.kv_from_start, c.ple_dim
    hc.attention_scale, hc.value_norm = c.attention_scale, c.value_norm
    keep = []
    for field, vals, dt in (("sliding_pattern", c.sliding_pattern, np.uint8), ("ff_dims", c.ff_dims, np.uint32),
                            ("kv_head_counts", c.kv_head_counts, np.uint32)):
        if len(vals):
            a = np.ascontiguousarray(vals, dtype=dt)
            keep.append(a)
            setattr(hc, field, a.ctypes.data)
    names = [t.name.encode() for t in table]
    arr = (_lib.HipTensor * len(table))()
    for i, t in enumerate(table):
        arr[i] = _lib.HipTensor(names[i], t.type, t.rows, t.cols, t.data.ctypes.data)
    return hc, arr, (names, keep)


def estimate(source, max_context: int = 0) -> dict:
    """Device bytes a session would take (brisk_hip_session_estimate; nothing is allocated, no GPU needed)."""
    L = _lib.load()
    if isinstance(source, str):
        source = _model.load(source)
    _, c, table = source
    hc, arr, keep = _c_args(c, table)
    m = _lib.HipMemory()
    _lib.check(L.brisk_hip_session_estimate(C.byref(hc), arr, len(table), max_context, C.byref(m)))
    return {"weights": m.weights, "cache": m.cache, "scratch": m.scratch, "total": m.total}


def device_memory(device: int = 0):
    """(free, total) bytes of the device (brisk_hip_device_memory)."""
    L = _lib.load()
    f, t = C.c_size_t(), C.c_size_t()
    _lib.check(L.brisk_hip_device_memory(device, C.byref(f), C.byref(t)))
    return f.value, t.value


class HipSession:
    """One sequence on one GPU.  ``source`` is a GGUF path or a (GgufFile, ModelConfig, table) triple."""

    max_scored_tokens = 64  # Engine::kMaxScoredTokens

    # Sessions still open when the interpreter exits are closed by an atexit hook, which runs
    # before the HIP runtime's own exit handlers (a session destroyed after them would free
    # streams and pinned buffers of a runtime already torn down).
    _live = weakref.WeakSet()

    def __init__(self, source, max_context: int = 0, device: int = 0):
        L = _lib.load()
        self._L = L
        if isinstance(source, str):
            source = _model.load(source)
        self.file, self.config, table = source
        c = self.config
        hc, arr, keep = _c_args(c, table)
        h = C.c_void_p()
        _lib.check(L.brisk_hip_session_create(C.byref(hc), arr, len(table), max_context, device, C.byref(h)))
        self._h = h
        self.vocab = c.vocab
        HipSession._live.add(self)

    def close(self):
        if getattr(self, "_h", None):
            self._L.brisk_hip_session_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def _tokens(tokens) -> np.ndarray:
        return np.ascontiguousarray(np.atleast_1d(np.asarray(tokens)), dtype=np.int32)

    def eval(self, tokens, logits: bool = True):
        t = self._tokens(tokens)
        out = np.empty(self.vocab, np.float32) if logits else None
        _lib.check(self._L.brisk_hip_session_eval(self._h, _ptr(t), len(t), _ptr(out) if logits else None))
        return out

    def eval_all(self, tokens) -> np.ndarray:
        t = self._tokens(tokens)
        out = np.empty((len(t), self.vocab), np.float32)
        _lib.check(self._L.brisk_hip_session_eval_all(self._h, _ptr(t), len(t), _ptr(out)))
        return out

    def eval_greedy(self, tokens) -> int:
        t = self._tokens(tokens)
        nxt = C.c_int32()
        _lib.check(self._L.brisk_hip_session_eval_greedy(self._h, _ptr(t), len(t), C.byref(nxt)))
        return int(nxt.value)

    def generate(self, prompt, n_gen: int) -> np.ndarray:
        p = self._tokens(prompt)
        out = np.zeros(n_gen, np.int32)
        _lib.check(self._L.brisk_hip_session_generate(self._h, _ptr(p), len(p), n_gen, _ptr(out)))
        return out

    def decode(self, n: int, ids: bool = True):
        """n more greedy steps from the pending pick; returns the n new ids (or None)."""
        out = np.zeros(n, np.int32) if ids else None
        _lib.check(self._L.brisk_hip_session_decode(self._h, n, _ptr(out) if ids else None))
        return out

    def rollback(self, position: int):
        _lib.check(self._L.brisk_hip_session_rollback(self._h, position))

    @property
    def position(self) -> int:
        return self._L.brisk_hip_session_position(self._h)

    @property
    def max_context(self) -> int:
        return self._L.brisk_hip_session_max_context(self._h)

    def kv_cache(self, layer: int, value: bool):
        """(device pointer, bytes) of a layer's fp16 cache [kv_heads][max_context][head_dim]."""
        p, n = C.c_void_p(), C.c_size_t()
        _lib.check(self._L.brisk_hip_session_kv_cache(self._h, layer, int(value), C.byref(p), C.byref(n)))
        return p.value, n.value

    def set_position(self, position: int):
        _lib.check(self._L.brisk_hip_session_set_position(self._h, position))

    @property
    def stream(self) -> int:
        return self._L.brisk_hip_session_stream(self._h)

    def log_likelihood(self, tokens, chunk: int = 64) -> float:
        """Engine::log_likelihood (src/engine.cpp:10-33): sum of log p(tokens[i] | tokens[:i]), i >= 1."""
        t = self._tokens(tokens)
        if len(t) < 2:
            raise RuntimeError("need at least two tokens to score")
        chunk = max(1, min(chunk, self.max_scored_tokens))
        total = 0.0
        for begin in range(0, len(t), chunk):
            n = min(chunk, len(t) - begin)
            logits = self.eval_all(t[begin:begin + n])
            for i in range(n):
                if begin + i + 1 >= len(t):
                    break
                row = logits[i].astype(np.float64)
                mx = row.max()
                total += (row[t[begin + i + 1]] - mx) - np.log(np.exp(row - mx).sum())
        return total


@atexit.register
def _close_live_sessions():
    for s in list(HipSession._live):
        s.close()
