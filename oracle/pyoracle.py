"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU oracle.

``Oracle`` wraps oracle/_build/liboracle.so (the C restatement in oracle.c);
``Reference`` wraps oracle/_ref/libbrisk_ref.so (the reference's own engine,
compiled from its sources by oracle/Makefile).  Only tests/, the smoke check and
bench.py's cpu_baseline leg import this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libbrisk_ref.so")

_vp, _sz, _i, _f, _u16 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_uint16


class OracleConfig(C.Structure):
    _fields_ = [("arch", C.c_int), ("embd", C.c_int), ("layers", C.c_int), ("heads", C.c_int),
                ("kv_heads", C.c_int), ("head_dim", C.c_int), ("ff", C.c_int), ("vocab", C.c_int),
                ("rope_base", C.c_float), ("eps", C.c_float), ("max_context", C.c_int),
                ("sliding_window", C.c_int), ("rope_base_local", C.c_float), ("rope_scale", C.c_float),
                ("final_softcap", C.c_float), ("rope_dim", C.c_int), ("rope_attn_factor", C.c_float),
                ("rope_original_context", C.c_int), ("conv_taps", C.c_int), ("ssm_state", C.c_int),
                ("ssm_k_heads", C.c_int), ("ssm_v_heads", C.c_int), ("ssm_inner", C.c_int), ("ssm_conv", C.c_int),
                ("head_dim_local", C.c_int), ("kv_from_start", C.c_int), ("ple_dim", C.c_int), ("value_norm", C.c_int),
                ("attention_scale", C.c_float), ("sliding_pattern", C.c_void_p), ("ff_dims", C.c_void_p),
                ("kv_head_counts", C.c_void_p)]


class OracleTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("rows", C.c_uint64), ("cols", C.c_uint64),
                ("data", C.c_void_p)]


def ptr(a: np.ndarray):
    return a.ctypes.data_as(_vp)


_oracle = None
_ref = None


def build():
    """Builds the oracle (and, where the reference tree exists, oracle/_ref)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def oracle_lib():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = C.CDLL(ORACLE_SO)
        L.or_half_to_float.argtypes = [_u16]
        L.or_half_to_float.restype = _f
        L.or_float_to_half.argtypes = [_f]
        L.or_float_to_half.restype = _u16
        L.or_quantize_q8_0.argtypes = [_vp, _vp, _sz]
        L.or_quantize_q8_k.argtypes = [_vp, _vp, _sz, _i]
        L.or_dot.argtypes = [_i, _i, _vp, _vp, _sz]
        L.or_dot.restype = _f
        L.or_matvec.argtypes = [_i, _vp, _sz, _sz, _vp, _vp]
        L.or_dequantize.argtypes = [_i, _vp, _vp, _sz]
        L.or_repack_tq2_0x16.argtypes = [_vp, _sz, _sz, _vp]
        L.or_dot_f32.argtypes = [_vp, _vp, _sz]
        L.or_dot_f32.restype = _f
        L.or_softmax.argtypes = [_vp, _sz]
        L.or_rms_norm.argtypes = [_vp, _vp, _f, _vp, _sz]
        L.or_expf_batch.argtypes = [_vp, _vp, _sz]
        L.or_expf_check.argtypes = [C.c_uint32, C.POINTER(C.c_uint64)]
        L.or_expf_check.restype = C.c_uint64
        L.or_tanhf_batch.argtypes = [_vp, _vp, _sz]
        L.or_tanhf_check.argtypes = [C.c_uint32, C.POINTER(C.c_uint64)]
        L.or_tanhf_check.restype = C.c_uint64
        L.or_log1pf_batch.argtypes = [_vp, _vp, _sz]
        L.or_log1pf_check.argtypes = [C.c_uint32, C.POINTER(C.c_uint64)]
        L.or_log1pf_check.restype = C.c_uint64
        L.or_activation_bits.argtypes = [_i, _sz]
        L.or_activation_bits.restype = _i
        L.or_session_create.argtypes = [C.POINTER(OracleConfig), C.POINTER(OracleTensor), _sz]
        L.or_session_create.restype = _vp
        L.or_session_destroy.argtypes = [_vp]
        L.or_session_eval.argtypes = [_vp, _vp, _sz, _i, _vp]
        L.or_session_position.argtypes = [_vp]
        L.or_session_position.restype = _sz
        L.or_session_rollback.argtypes = [_vp, _sz]
        L.or_session_kv.argtypes = [_vp, _i, _i]
        L.or_session_kv.restype = C.POINTER(C.c_uint16)
        L.or_session_set_position.argtypes = [_vp, _sz]
        L.or_last_error.restype = C.c_char_p
        _oracle = L
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref_lib():
    global _ref
    if _ref is None:
        L = C.CDLL(REF_SO)
        L.ref_open.argtypes = [C.c_char_p, _i, _sz]
        L.ref_open.restype = _vp
        L.ref_close.argtypes = [_vp]
        L.ref_vocab.argtypes = [_vp]
        L.ref_vocab.restype = C.c_uint32
        L.ref_position.argtypes = [_vp]
        L.ref_position.restype = _sz
        L.ref_rollback.argtypes = [_vp, _sz]
        L.ref_eval.argtypes = [_vp, _vp, _sz, _vp]
        L.ref_eval_all.argtypes = [_vp, _vp, _sz, _vp]
        L.ref_log_likelihood.argtypes = [_vp, _vp, _sz, C.POINTER(C.c_double)]
        L.ref_generate.argtypes = [_vp, _vp, _sz, _sz, _vp, _vp, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        L.ref_last_error.restype = C.c_char_p
        L.ref_half_to_float.argtypes = [_u16]
        L.ref_half_to_float.restype = _f
        L.ref_float_to_half.argtypes = [_f]
        L.ref_float_to_half.restype = _u16
        L.ref_quantize_q8_0.argtypes = [_vp, _vp, _sz]
        L.ref_quantize_q8_k.argtypes = [_vp, _vp, _sz, _i]
        L.ref_matvec.argtypes = [_i, _vp, _sz, _sz, _vp, _vp]
        L.ref_matmul.argtypes = [_i, _vp, _sz, _sz, _vp, _sz, _vp, _sz]
        L.ref_repack_tq2_0x16.argtypes = [_vp, _sz, _sz, _vp]
        L.ref_dequantize.argtypes = [_i, _vp, _vp, _sz]
        L.ref_softmax.argtypes = [_vp, _sz]
        L.ref_dot_f32.argtypes = [_vp, _vp, _sz]
        L.ref_dot_f32.restype = _f
        L.ref_config.argtypes = [_vp, C.POINTER(RefConfig)]
        _ref = L
    return _ref


class Oracle:
    """The C restatement's session over a tensor table (brisk_hip.model.tensor_table)."""

    def __init__(self, cfg, table, max_context: int):
        L = oracle_lib()
        self.L, self.cfg, self.max_context = L, cfg, max_context
        c = OracleConfig(cfg.arch, cfg.embd, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.ff, cfg.vocab,
                         cfg.rope_base, cfg.eps, max_context, cfg.sliding_window, cfg.rope_base_local, cfg.rope_scale,
                         cfg.final_softcap, cfg.rope_dim, cfg.rope_attn_factor, cfg.rope_original_context, cfg.conv_taps,
                         cfg.ssm_state, cfg.ssm_k_heads, cfg.ssm_v_heads, cfg.ssm_inner, cfg.ssm_conv)
        c.head_dim_local, c.kv_from_start, c.ple_dim = cfg.head_dim_local, cfg.kv_from_start, cfg.ple_dim
        c.value_norm, c.attention_scale = cfg.value_norm, cfg.attention_scale
        self._tables = []
        for field, vals, dt in (("sliding_pattern", cfg.sliding_pattern, np.uint8), ("ff_dims", cfg.ff_dims, np.int32),
                                ("kv_head_counts", cfg.kv_head_counts, np.int32)):
            if len(vals):
                a = np.ascontiguousarray(vals, dtype=dt)
                self._tables.append(a)
                setattr(c, field, a.ctypes.data)
        self._names = [t.name.encode() for t in table]
        arr = (OracleTensor * len(table))()
        for i, t in enumerate(table):
            arr[i] = OracleTensor(self._names[i], t.type, t.rows, t.cols, t.data.ctypes.data)
        self._keep = (table, arr)
        self.h = L.or_session_create(C.byref(c), arr, len(table))
        if not self.h:
            raise RuntimeError(L.or_last_error().decode())

    def close(self):
        if self.h:
            self.L.or_session_destroy(self.h)
            self.h = None

    __del__ = close

    def eval(self, tokens, all_logits=False) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((len(tokens) if all_logits else 1, self.cfg.vocab), np.float32)
        if self.L.or_session_eval(self.h, ptr(tokens), len(tokens), int(all_logits), ptr(out)) != 0:
            raise RuntimeError(self.L.or_last_error().decode())
        return out if all_logits else out[0]

    @property
    def position(self) -> int:
        return self.L.or_session_position(self.h)

    def rollback(self, p: int):
        if self.L.or_session_rollback(self.h, p) != 0:
            raise RuntimeError(self.L.or_last_error().decode())

    def kv(self, layer: int, value: bool) -> np.ndarray:
        """Layer ``layer``'s fp16-bit cache [kv_heads][max_context][head_dim], writable in place."""
        n = self.cfg.kv_heads * self.max_context * self.cfg.head_dim
        p = self.L.or_session_kv(self.h, layer, int(value))
        return np.ctypeslib.as_array(p, shape=(n,)).reshape(self.cfg.kv_heads, self.max_context, self.cfg.head_dim)

    def set_position(self, p: int):
        self.L.or_session_set_position(self.h, p)

    def generate(self, prompt, n_gen: int):
        """Greedy ids and top-1 minus top-2 gaps, as the reference's generate loop."""
        logits = self.eval(prompt)
        ids, gaps = [], []
        for i in range(n_gen):
            nxt = int(np.argmax(logits))
            ids.append(nxt)
            gaps.append(_gap(logits, nxt))
            if i + 1 == n_gen:
                break
            logits = self.eval([nxt])
        return np.array(ids, np.int32), np.array(gaps, np.float32)


def _gap(logits, best):
    second = np.max(np.delete(logits, best))
    return float(logits[best] - second)


class RefConfig(C.Structure):
    """ref_shim.cpp's RefConfig: the reference's ModelConfig (src/model.h:34-125) as parsed from a file."""
    _fields_ = [(n, C.c_uint32) for n in ("arch", "vocab", "embd", "layers", "heads", "kv_heads", "head_dim", "ff", "context")] + [
        ("rope_base", C.c_float), ("eps", C.c_float), ("rope_neox", C.c_int32), ("rope_dim", C.c_uint32),
        ("rope_original_context", C.c_uint32), ("rope_attn_factor", C.c_float), ("sliding_window", C.c_uint32),
        ("rope_base_local", C.c_float), ("rope_scale", C.c_float), ("embedding_scale", C.c_float),
        ("final_softcap", C.c_float), ("gelu", C.c_int32), ("conv_taps", C.c_uint32), ("no_rope_step", C.c_uint32),
        ("n_rope_factors", C.c_uint32), ("n_factors_short", C.c_uint32), ("n_factors_long", C.c_uint32),
        ("conv_layers", C.c_uint64), ("ssm_state", C.c_uint32), ("ssm_k_heads", C.c_uint32),
        ("ssm_v_heads", C.c_uint32), ("ssm_inner", C.c_uint32), ("ssm_conv", C.c_uint32), ("attention_gate", C.c_int32),
        ("recurrent_layers", C.c_uint64), ("head_dim_local", C.c_uint32), ("kv_from_start", C.c_uint32),
        ("ple_dim", C.c_uint32), ("attention_scale", C.c_float), ("value_norm", C.c_int32), ("sliding_layers", C.c_uint64),
        ("head_dim_of", C.c_uint32 * 64), ("kv_heads_of", C.c_uint32 * 64), ("ff_of", C.c_uint32 * 64),
        ("kv_layer_of", C.c_uint32 * 64)]


# the reference's Architecture enumerators (src/model.h:20-31), by GGUF architecture name
REF_ARCH = {"qwen3": 0, "qwen2": 1, "llama": 2, "gemma3": 3, "gemma4": 4, "bitnet": 5, "bitnet-b1.58": 5, "phi3": 6,
            "lfm2": 7, "smollm3": 8, "qwen35": 9}


class Reference:
    """The reference's own CPU Session (oracle/_ref), opened on a GGUF path."""

    def __init__(self, path: str, threads: int = 1, max_context: int = 1024):
        L = ref_lib()
        self.L = L
        self.h = L.ref_open(path.encode(), threads, max_context)
        if not self.h:
            raise RuntimeError(L.ref_last_error().decode())
        self.vocab = L.ref_vocab(self.h)

    def close(self):
        if self.h:
            self.L.ref_close(self.h)
            self.h = None

    __del__ = close

    def config(self) -> RefConfig:
        out = RefConfig()
        if self.L.ref_config(self.h, C.byref(out)) != 0:
            raise RuntimeError(self.L.ref_last_error().decode())
        return out

    def eval(self, tokens) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab, np.float32)
        if self.L.ref_eval(self.h, ptr(tokens), len(tokens), ptr(out)) != 0:
            raise RuntimeError(self.L.ref_last_error().decode())
        return out

    def eval_all(self, tokens) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((len(tokens), self.vocab), np.float32)
        if self.L.ref_eval_all(self.h, ptr(tokens), len(tokens), ptr(out)) != 0:
            raise RuntimeError(self.L.ref_last_error().decode())
        return out

    @property
    def position(self) -> int:
        return self.L.ref_position(self.h)

    def rollback(self, p: int):
        if self.L.ref_rollback(self.h, p) != 0:
            raise RuntimeError(self.L.ref_last_error().decode())

    def log_likelihood(self, tokens) -> float:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = C.c_double()
        if self.L.ref_log_likelihood(self.h, ptr(tokens), len(tokens), C.byref(out)) != 0:
            raise RuntimeError(self.L.ref_last_error().decode())
        return out.value

    def generate(self, prompt, n_gen: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        ids = np.zeros(n_gen, np.int32)
        gaps = np.zeros(n_gen, np.float32)
        a, b = C.c_double(), C.c_double()
        if self.L.ref_generate(self.h, ptr(prompt), len(prompt), n_gen, ptr(ids), ptr(gaps), C.byref(a), C.byref(b)) != 0:
            raise RuntimeError(self.L.ref_last_error().decode())
        return ids, gaps, a.value, b.value


# ---------------------------------------------------------------- the drop-in binding, driven as the reference drives an Engine

HIP_ENGINE_PATH = os.path.join(HERE, "_ref", "libhip_engine.so")
HIP_ENGINE_EXPORTS = ("he_last_error", "he_open", "he_close", "he_position", "he_rollback", "he_eval", "he_eval_all",
                      "he_generate", "he_generate_greedy", "he_speculative", "he_serve_warmup", "he_serve_prefill",
                      "he_serve_extend", "he_log_likelihood")


def hip_engine_available() -> bool:
    return os.path.exists(HIP_ENGINE_PATH)


def hip_engine_lib():
    L = C.CDLL(HIP_ENGINE_PATH)
    vp, sz = C.c_void_p, C.c_size_t
    L.he_last_error.restype = C.c_char_p
    L.he_open.argtypes = [C.c_char_p, sz]
    L.he_open.restype = vp
    L.he_close.argtypes = [vp]
    L.he_position.argtypes = [vp]
    L.he_position.restype = sz
    L.he_rollback.argtypes = [vp, sz]
    for f in (L.he_eval, L.he_eval_all, L.he_serve_extend):
        f.argtypes = [vp, vp, sz, vp]
    for f in (L.he_generate, L.he_generate_greedy):
        f.argtypes = [vp, vp, sz, sz, vp]
    L.he_speculative.argtypes = [vp, C.c_char_p, C.c_int, vp, sz, sz, sz, vp, vp]
    L.he_serve_warmup.argtypes = [vp, C.c_int32]
    L.he_serve_prefill.argtypes = [vp, vp, sz, vp, C.POINTER(sz)]
    L.he_log_likelihood.argtypes = [vp, vp, sz, C.POINTER(C.c_double)]
    return L


class HipEngine:
    """HipSession : Engine (brisk-llm_amd/binding/hip_session.h) over Model(file, repack = false), through
    oracle/_ref/libhip_engine.so: the calls the reference's CLI, server and speculative driver make."""

    def __init__(self, path: str, max_context: int, vocab: int):
        self.L = hip_engine_lib()
        self.vocab = vocab
        self.h = self.L.he_open(path.encode(), max_context)
        if not self.h:
            raise RuntimeError(self.L.he_last_error().decode())

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.L.he_last_error().decode())

    def close(self):
        if self.h:
            self.L.he_close(self.h)
            self.h = None

    __del__ = close

    @property
    def position(self) -> int:
        return self.L.he_position(self.h)

    def rollback(self, p: int):
        self._check(self.L.he_rollback(self.h, p))

    def eval(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab, np.float32)
        self._check(self.L.he_eval(self.h, ptr(t), len(t), ptr(out)))
        return out

    def eval_all(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((len(t), self.vocab), np.float32)
        self._check(self.L.he_eval_all(self.h, ptr(t), len(t), ptr(out)))
        return out

    def generate(self, prompt, n_gen: int, on_device: bool = False) -> np.ndarray:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, np.int32)
        f = self.L.he_generate_greedy if on_device else self.L.he_generate
        self._check(f(self.h, ptr(p), len(p), n_gen, ptr(out)))
        return out

    def speculative(self, prompt, n_gen: int, draft_tokens: int, draft_path=None, threads: int = 1):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, np.int32)
        stats = np.zeros(4, np.uint64)
        self._check(self.L.he_speculative(self.h, draft_path.encode() if draft_path else None, threads, ptr(p), len(p), n_gen,
                                          draft_tokens, ptr(out), ptr(stats)))
        return out, dict(zip(("rounds", "plain", "drafted", "accepted"), map(int, stats)))

    def serve_warmup(self, first: int):
        self._check(self.L.he_serve_warmup(self.h, first))

    def serve_prefill(self, prompt):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(self.vocab, np.float32)
        reused = C.c_size_t()
        self._check(self.L.he_serve_prefill(self.h, ptr(p), len(p), ptr(out), C.byref(reused)))
        return out, reused.value

    def serve_extend(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab, np.float32)
        self._check(self.L.he_serve_extend(self.h, ptr(t), len(t), ptr(out)))
        return out

    def log_likelihood(self, tokens) -> float:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = C.c_double()
        self._check(self.L.he_log_likelihood(self.h, ptr(t), len(t), C.byref(out)))
        return out.value
