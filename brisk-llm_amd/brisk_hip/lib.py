"""ctypes binding of libbrisk_hip.so (include/brisk_hip.h).

The library is the product: this module only loads it and declares the
signatures.  There is no fallback — if the library is missing or a call
fails, the error propagates.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbrisk_hip.so")

_vp, _sz, _i, _f = C.c_void_p, C.c_size_t, C.c_int, C.c_float

# Expected exports of include/brisk_hip.h (checked by tests/test_abi.py).
EXPORTS = (
    "brisk_hip_last_error", "brisk_hip_abi_version", "brisk_hip_device_count", "brisk_hip_packed_bytes", "brisk_hip_pack",
    "brisk_hip_quantize_q8_0", "brisk_hip_quantize_q8_k", "brisk_hip_matvec", "brisk_hip_matmul", "brisk_hip_matmul_noalloc", "brisk_hip_gemv", "brisk_hip_expf", "brisk_hip_tanhf", "brisk_hip_log1pf",
    "brisk_hip_div_selftest", "brisk_hip_mfma_rate",
    "brisk_hip_session_estimate", "brisk_hip_device_memory", "brisk_hip_session_create", "brisk_hip_session_destroy", "brisk_hip_session_eval", "brisk_hip_session_eval_all",
    "brisk_hip_session_eval_greedy", "brisk_hip_session_generate", "brisk_hip_session_decode", "brisk_hip_session_rollback",
    "brisk_hip_session_position", "brisk_hip_session_max_context", "brisk_hip_session_kv_cache",
    "brisk_hip_session_set_position", "brisk_hip_session_stream", "brisk_hip_session_trace",
)


class HipConfig(C.Structure):
    _fields_ = [("arch", C.c_int), ("vocab", C.c_uint32), ("embd", C.c_uint32), ("layers", C.c_uint32),
                ("heads", C.c_uint32), ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("ff", C.c_uint32),
                ("context_length", C.c_uint32), ("rope_base", C.c_float), ("rms_epsilon", C.c_float),
                ("sliding_window", C.c_uint32), ("rope_base_local", C.c_float), ("rope_scale", C.c_float),
                ("final_softcap", C.c_float), ("rope_dim", C.c_uint32), ("rope_attn_factor", C.c_float),
                ("rope_original_context", C.c_uint32), ("conv_taps", C.c_uint32), ("rope_neox", C.c_int32),
                ("no_rope_step", C.c_uint32), ("embedding_scale", C.c_float), ("gelu", C.c_int32),
                ("ssm_state", C.c_uint32), ("ssm_k_heads", C.c_uint32), ("ssm_v_heads", C.c_uint32),
                ("ssm_inner", C.c_uint32), ("ssm_conv", C.c_uint32), ("head_dim_local", C.c_uint32),
                ("kv_from_start", C.c_uint32), ("ple_dim", C.c_uint32), ("attention_scale", C.c_float),
                ("value_norm", C.c_int32), ("sliding_pattern", C.c_void_p), ("ff_dims", C.c_void_p),
                ("kv_head_counts", C.c_void_p)]


class HipTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("rows", C.c_uint64), ("cols", C.c_uint64), ("data", C.c_void_p)]


class HipMemory(C.Structure):
    _fields_ = [("weights", C.c_size_t), ("cache", C.c_size_t), ("scratch", C.c_size_t), ("total", C.c_size_t)]


class BriskHipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_lib = None


def load():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
    L = C.CDLL(LIB_PATH)
    L.brisk_hip_last_error.restype = C.c_char_p
    L.brisk_hip_device_count.argtypes = [C.POINTER(C.c_int)]
    L.brisk_hip_packed_bytes.argtypes = [_i, _sz, _sz]
    L.brisk_hip_packed_bytes.restype = _sz
    L.brisk_hip_pack.argtypes = [_i, _vp, _sz, _sz, _vp, _vp]
    L.brisk_hip_quantize_q8_0.argtypes = [_vp, _vp, _sz, _vp]
    L.brisk_hip_quantize_q8_k.argtypes = [_vp, _vp, _sz, _i, _vp]
    L.brisk_hip_matvec.argtypes = [_i, _i, _vp, _sz, _sz, _vp, _vp, _vp]
    L.brisk_hip_matmul.argtypes = [_i, _i, _vp, _sz, _sz, _vp, _sz, _vp, _sz, _vp]
    L.brisk_hip_matmul_noalloc.argtypes = [_i, _i, _vp, _sz, _sz, _vp, _sz, _vp, _sz, _vp]
    L.brisk_hip_gemv.argtypes = [_i, _i, _vp, _sz, _sz, _vp, _vp, _f, _vp, _i, _vp]
    L.brisk_hip_expf.argtypes = [_vp, _vp, _sz, _vp]
    L.brisk_hip_tanhf.argtypes = [_vp, _vp, _sz, _vp]
    L.brisk_hip_log1pf.argtypes = [_vp, _vp, _sz, _vp]
    L.brisk_hip_div_selftest.argtypes = [C.POINTER(C.c_ulonglong)]
    L.brisk_hip_mfma_rate.argtypes = [_i, C.POINTER(C.c_double)]
    L.brisk_hip_session_estimate.argtypes = [C.POINTER(HipConfig), C.POINTER(HipTensor), _sz, _sz, C.POINTER(HipMemory)]
    L.brisk_hip_device_memory.argtypes = [_i, C.POINTER(_sz), C.POINTER(_sz)]
    L.brisk_hip_session_create.argtypes = [C.POINTER(HipConfig), C.POINTER(HipTensor), _sz, _sz, _i, C.POINTER(_vp)]
    L.brisk_hip_session_destroy.argtypes = [_vp]
    L.brisk_hip_session_eval.argtypes = [_vp, _vp, _sz, _vp]
    L.brisk_hip_session_eval_all.argtypes = [_vp, _vp, _sz, _vp]
    L.brisk_hip_session_eval_greedy.argtypes = [_vp, _vp, _sz, C.POINTER(C.c_int32)]
    L.brisk_hip_session_generate.argtypes = [_vp, _vp, _sz, _sz, _vp]
    L.brisk_hip_session_decode.argtypes = [_vp, _sz, _vp]
    L.brisk_hip_session_rollback.argtypes = [_vp, _sz]
    L.brisk_hip_session_position.argtypes = [_vp]
    L.brisk_hip_session_position.restype = _sz
    L.brisk_hip_session_max_context.argtypes = [_vp]
    L.brisk_hip_session_max_context.restype = _sz
    L.brisk_hip_session_kv_cache.argtypes = [_vp, _i, _i, C.POINTER(_vp), C.POINTER(_sz)]
    L.brisk_hip_session_set_position.argtypes = [_vp, _sz]
    L.brisk_hip_session_stream.argtypes = [_vp]
    L.brisk_hip_session_stream.restype = _vp
    L.brisk_hip_session_trace.argtypes = [_vp, C.POINTER(C.c_ulonglong), _sz]
    L.brisk_hip_session_trace.restype = _sz
    _lib = L
    return L


def check(rc: int):
    if rc != 0:
        raise BriskHipError(rc, load().brisk_hip_last_error().decode())
