"""Model configuration and tensor table from a GGUF file (host side).

Restates the part of the reference's loader the HIP session needs:
``Model::parse_config`` (src/model.cpp:161-301) for the families the HIP
session runs (qwen3, llama, bitnet, qwen2, smollm3, gemma3, gemma4, phi3, lfm2, qwen35), the tensor names and shapes of
``Model::Model`` (src/model.cpp:303-423) and the tied output projection
(src/model.cpp:328-330).  The session takes the weights as GGUF-layout bytes,
as the reference's ``Model(file, repack = false)`` hands them to a GPU session.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import gguf as G

ARCH_QWEN3, ARCH_LLAMA, ARCH_BITNET, ARCH_QWEN2, ARCH_SMOLLM3, ARCH_GEMMA3, ARCH_PHI3, ARCH_LFM2, ARCH_QWEN35, ARCH_GEMMA4 = range(10)
_ARCH = {"qwen3": ARCH_QWEN3, "llama": ARCH_LLAMA, "bitnet": ARCH_BITNET, "bitnet-b1.58": ARCH_BITNET,
         "qwen2": ARCH_QWEN2, "smollm3": ARCH_SMOLLM3, "gemma3": ARCH_GEMMA3, "phi3": ARCH_PHI3,
         "lfm2": ARCH_LFM2, "qwen35": ARCH_QWEN35, "gemma4": ARCH_GEMMA4}
QUANT_TYPES = (G.T_Q4_0, G.T_Q4_1, G.T_Q5_0, G.T_Q8_0, G.T_Q4_K, G.T_Q5_K, G.T_Q6_K, G.T_TQ2_0)


class ModelError(RuntimeError):
    pass


def fail(what: str):
    raise ModelError("model: " + what)  # src/model.cpp:18


@dataclass
class ModelConfig:
    arch: int
    arch_name: str
    vocab: int
    embd: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    ff: int
    context: int
    rope_base: float
    eps: float
    # Gemma 3 (src/model.cpp:170-176); zero for the other families
    sliding_window: int = 0
    rope_base_local: float = 0.0
    rope_scale: float = 0.0
    final_softcap: float = 0.0
    # Phi-3 (src/model.cpp:177-187); zero for the other families
    rope_dim: int = 0
    rope_attn_factor: float = 0.0
    rope_original_context: int = 0
    # LFM2 (src/model.cpp:229-253): convolution width; layers whose head_count_kv entry is 0 convolve
    conv_taps: int = 0
    conv_layers: tuple = ()
    # Qwen3.5 (src/model.cpp:254-274): Gated DeltaNet state size, key/value heads, inner width and
    # conv width; layers whose head_count_kv entry is 0 (every layer but each interval-th) are recurrent
    ssm_state: int = 0
    ssm_k_heads: int = 0
    ssm_v_heads: int = 0
    ssm_inner: int = 0
    ssm_conv: int = 0
    recurrent_layers: tuple = ()
    # Gemma 4 (src/model.cpp:189-226): the sliding layers' head size (0: head_dim), the first layer
    # that reads an earlier layer's K/V (0: none), the per-layer embedding width, the score scale
    # (0: 1 / sqrt(head size)), V's weightless norm; per-layer tables (empty: the rule / the scalar)
    head_dim_local: int = 0
    kv_from_start: int = 0
    ple_dim: int = 0
    attention_scale: float = 0.0
    value_norm: int = 0
    sliding_pattern: tuple = ()
    ff_dims: tuple = ()
    kv_head_counts: tuple = ()

    def layer_slides(self, layer: int) -> bool:  # src/model.h:87-90
        if self.sliding_pattern:
            return bool(self.sliding_pattern[layer])
        return self.sliding_window != 0 and layer % 6 != 5

    def head_dim_of(self, layer: int) -> int:  # src/model.h:111-113
        return self.head_dim_local if self.head_dim_local and self.layer_slides(layer) else self.head_dim

    def kv_heads_of(self, layer: int) -> int:  # src/model.h:91-93
        return int(self.kv_head_counts[layer]) if self.kv_head_counts else self.kv_heads

    def ff_of(self, layer: int) -> int:  # src/model.h:118
        return int(self.ff_dims[layer]) if self.ff_dims else self.ff

    def kv_layer_of(self, layer: int) -> int:  # src/model.h:114-117
        if self.kv_from_start == 0 or layer < self.kv_from_start:
            return layer
        return self.kv_from_start - (2 if self.layer_slides(layer) else 1)

    @property
    def ssm_qkv_dim(self) -> int:  # src/model.h:108
        return 2 * self.ssm_k_heads * self.ssm_state + self.ssm_inner

    @property
    def rope_neox(self) -> bool:  # src/model.cpp:167
        return self.arch not in (ARCH_LLAMA, ARCH_SMOLLM3)

    def layer_has_rope(self, layer: int) -> bool:  # src/model.h:110; SmolLM3's step of 4, src/model.cpp:168
        return not (self.arch == ARCH_SMOLLM3 and (layer + 1) % 4 == 0)

    @property
    def query_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


def parse_config(f: G.GgufFile) -> ModelConfig:
    name = f.get("general.architecture")
    if name not in _ARCH:
        fail(f"unsupported architecture '{name}'; the HIP session runs qwen3, qwen2, llama, smollm3, gemma3, gemma4, "
             "phi3, lfm2, qwen35 and bitnet")
    p = name + "."

    def u32(key):
        v = f.get(p + key)
        if v is None:
            fail(f"missing metadata '{p + key}'")
        return int(v)

    def f32(key):
        v = f.get(p + key)
        if v is None:
            fail(f"missing metadata '{p + key}'")
        return float(v)

    embd, layers, heads = u32("embedding_length"), u32("block_count"), u32("attention.head_count")
    kv_raw = f.get(p + "attention.head_count_kv")
    per_layer_kv = list(kv_raw) if isinstance(kv_raw, (list, tuple)) else None  # per layer (src/model.cpp:229-238)
    if name == "qwen35" and per_layer_kv is None:  # every interval-th layer attends (src/model.cpp:255-271)
        interval = int(f.get(p + "full_attention_interval", 0))
        if interval == 0:
            fail("qwen35: full_attention_interval is missing")
        per_layer_kv = [int(kv_raw or 0) if (l + 1) % interval == 0 else 0 for l in range(layers)]
    if per_layer_kv is not None and len(per_layer_kv) != layers:
        fail("head_count_kv array length")
    if per_layer_kv is not None and len({k for k in per_layer_kv if k != 0}) > 1 and name != "gemma4":
        # one head count for every attention layer but Gemma 4's (kv_head_count_of, src/model.h:91)
        fail("attention layers with different key/value head counts are not supported")
    kv = int(max(per_layer_kv)) if per_layer_kv is not None else u32("attention.head_count_kv")
    ff_raw = f.get(p + "feed_forward_length")
    ff_dims = ()
    if name == "gemma4" and isinstance(ff_raw, (list, tuple)):  # per layer (src/model.cpp:202-212)
        if any(int(w) <= 0 for w in ff_raw):
            fail("non-positive feed-forward width")
        ff_dims = tuple(int(w) for w in ff_raw)
        if len(ff_dims) != layers:
            fail("feed_forward_length array length")
        ff = max(ff_dims)
    else:
        ff = u32("feed_forward_length")
    ctx = u32("context_length")
    if 0 in (embd, layers, heads, kv, ff, ctx):
        fail("a model dimension is zero")
    for k in (per_layer_kv if per_layer_kv is not None else [kv]):  # src/model.cpp:275-280
        if k == 0 and name in ("lfm2", "qwen35"):
            continue
        if k == 0 or heads % k:
            fail("head_count is not a multiple of head_count_kv")
        if heads // k > 16:
            fail("more than 16 query heads per key/value head is not supported")
    head_dim = int(f.get(p + "attention.key_length", embd // heads))
    if head_dim == 0 or head_dim % 32:
        fail("head size must be a non-zero multiple of 32")
    if int(f.get(p + "attention.value_length", head_dim)) != head_dim:
        fail("key and value head sizes differ")
    emb = f.tensor("token_embd.weight")
    if emb is None or len(emb.dims) != 2 or emb.dims[0] != embd:
        fail("missing or misshapen token_embd.weight")
    cfg = ModelConfig(_ARCH[name], name, int(emb.dims[1]), embd, layers, heads, kv, head_dim, ff, ctx,
                      f32("rope.freq_base"), f32("attention.layer_norm_rms_epsilon"))
    cfg.ff_dims = ff_dims
    if cfg.arch == ARCH_GEMMA4:  # src/model.cpp:189-226
        pattern = f.get(p + "attention.sliding_window_pattern")
        if pattern is not None:
            cfg.sliding_pattern = tuple(1 if b else 0 for b in pattern)
            if len(cfg.sliding_pattern) != layers:
                fail("sliding window pattern length")
        cfg.head_dim_local = int(f.get(p + "attention.key_length_swa", 0))
        if cfg.head_dim_local and (cfg.head_dim_local % 32 or cfg.head_dim_local > head_dim):
            fail("the sliding layers' head size must be a multiple of 32 no larger than the global one")
        shared = int(f.get(p + "attention.shared_kv_layers", 0))
        if shared:
            if shared + 2 > layers:
                fail("more shared K/V layers than layers")
            cfg.kv_from_start = layers - shared
        cfg.ple_dim = int(f.get(p + "embedding_length_per_layer_input", 0))
        cfg.attention_scale = 1.0
        cfg.value_norm = 1
        if per_layer_kv is not None:
            cfg.kv_head_counts = tuple(int(k) for k in per_layer_kv)
    if cfg.arch in (ARCH_GEMMA3, ARCH_GEMMA4):
        cfg.sliding_window = int(f.get(p + "attention.sliding_window", 0))
        cfg.rope_base_local = float(f.get(p + "rope.freq_base_swa", 10000.0))
        cfg.rope_scale = float(np.float32(1.0) / np.float32(f.get(p + "rope.scaling.factor", 1.0)))  # in float
        cfg.final_softcap = float(f.get(p + "final_logit_softcapping", 0.0))
    if cfg.arch == ARCH_LFM2:
        cfg.conv_taps = int(f.get(p + "shortconv.l_cache", 0))
        if not 2 <= cfg.conv_taps <= 8:
            fail("unsupported short-convolution width")
        cfg.conv_layers = tuple(l for l in range(layers) if per_layer_kv is not None and per_layer_kv[l] == 0)
    elif cfg.arch == ARCH_QWEN35:
        cfg.ssm_state, cfg.ssm_k_heads, cfg.ssm_v_heads = u32("ssm.state_size"), u32("ssm.group_count"), u32("ssm.time_step_rank")
        cfg.ssm_inner, cfg.ssm_conv = u32("ssm.inner_size"), u32("ssm.conv_kernel")
        if (cfg.ssm_v_heads == 0 or cfg.ssm_inner % cfg.ssm_v_heads or cfg.ssm_inner // cfg.ssm_v_heads != cfg.ssm_state
                or cfg.ssm_k_heads != cfg.ssm_v_heads or not 2 <= cfg.ssm_conv <= 8):
            fail("qwen35: unsupported DeltaNet shape (equal key and value heads of state_size values are supported)")
        if cfg.ssm_state > 256:
            fail("qwen35: a DeltaNet state wider than 256 is not supported")
        cfg.recurrent_layers = tuple(l for l in range(layers) if per_layer_kv[l] == 0)
        cfg.rope_dim = int(f.get(p + "rope.dimension_count", 0))
    elif per_layer_kv is not None and min(per_layer_kv) != kv and cfg.arch != ARCH_GEMMA4:
        fail("per-layer key/value head counts are not supported for this family")
    if cfg.arch == ARCH_PHI3:
        cfg.rope_dim = int(f.get(p + "rope.dimension_count", 0))
        cfg.rope_attn_factor = float(f.get(p + "rope.scaling.attn_factor", 1.0))
        cfg.rope_original_context = int(f.get(p + "rope.scaling.original_context_length", 0))
    return cfg


@dataclass
class TensorRef:
    name: str
    type: int
    rows: int
    cols: int
    data: object  # numpy uint8 view of the GGUF bytes


def tensor_table(f: G.GgufFile, cfg: ModelConfig) -> list:
    """Every tensor the forward step reads, shape-checked as src/model.cpp:426-478 does."""
    out = []

    def vec(name, n):
        t = f.tensor(name)
        if t is None:
            fail(f"missing tensor '{name}'")
        if t.n_elements() != n:
            fail(f"tensor '{name}' has an unexpected size")
        if t.type != G.T_F32:
            fail(f"tensor '{name}' has type {G.TYPE_NAMES.get(t.type, t.type)}; only F32 is supported here")
        out.append(TensorRef(name, t.type, 1, n, t.data))

    def mat(name, rows, cols):
        t = f.tensor(name)
        if t is None:
            fail(f"missing tensor '{name}'")
        if len(t.dims) != 2 or t.dims[0] != cols or t.dims[1] != rows:
            fail(f"tensor '{name}' has an unexpected shape")
        if t.type not in QUANT_TYPES:
            fail(f"tensor '{name}' has type {G.TYPE_NAMES.get(t.type, t.type)}, which the HIP session does not take")
        if cols % G.BLOCK[t.type][0]:
            fail(f"tensor '{name}' row length is not a multiple of its block size")
        out.append(TensorRef(name, t.type, rows, cols, t.data))

    e, qd, kvd = cfg.embd, cfg.query_dim, cfg.kv_dim
    mat("token_embd.weight", cfg.vocab, e)
    rd = cfg.rope_dim or cfg.head_dim
    if f.tensor("rope_freqs.weight") is not None:  # Llama 3's per-frequency factors (src/model.cpp:314-318)
        vec("rope_freqs.weight", cfg.head_dim // 2)
    if cfg.arch == ARCH_PHI3 and f.tensor("rope_factors_short.weight") is not None:  # LongRoPE (src/model.cpp:181-186)
        vec("rope_factors_short.weight", rd // 2)
        vec("rope_factors_long.weight", rd // 2)
    vec("token_embd_norm.weight" if cfg.arch == ARCH_LFM2 else "output_norm.weight", e)  # src/model.cpp:331
    if cfg.ple_dim:  # Gemma 4's per-layer embeddings (src/model.cpp:319-324)
        pall = cfg.ple_dim * cfg.layers
        mat("per_layer_token_embd.weight", cfg.vocab, pall)
        mat("per_layer_model_proj.weight", pall, e)
        vec("per_layer_proj_norm.weight", cfg.ple_dim)
    if f.tensor("output.weight") is not None:
        mat("output.weight", cfg.vocab, e)
    for l in range(cfg.layers):
        b = f"blk.{l}."
        vec(b + "attn_norm.weight", e)
        if l in cfg.recurrent_layers:  # Qwen3.5 Gated DeltaNet (src/model.cpp:343-358)
            mat(b + "attn_qkv.weight", cfg.ssm_qkv_dim, e)
            mat(b + "attn_gate.weight", cfg.ssm_inner, e)
            mat(b + "ssm_alpha.weight", cfg.ssm_v_heads, e)
            mat(b + "ssm_beta.weight", cfg.ssm_v_heads, e)
            vec(b + "ssm_a", cfg.ssm_v_heads)
            vec(b + "ssm_dt.bias", cfg.ssm_v_heads)
            vec(b + "ssm_conv1d.weight", cfg.ssm_conv * cfg.ssm_qkv_dim)
            vec(b + "ssm_norm.weight", cfg.ssm_state)
            mat(b + "ssm_out.weight", e, cfg.ssm_inner)
            vec(b + "post_attention_norm.weight", e)
            mat(b + "ffn_gate.weight", cfg.ff, e)
            mat(b + "ffn_up.weight", cfg.ff, e)
            mat(b + "ffn_down.weight", e, cfg.ff)
            continue
        if l in cfg.conv_layers:  # LFM2 short convolution (src/model.cpp:360-364)
            mat(b + "shortconv.in_proj.weight", 3 * e, e)
            mat(b + "shortconv.out_proj.weight", e, e)
            vec(b + "shortconv.conv.weight", cfg.conv_taps * e)
            vec(b + "ffn_norm.weight", e)
            mat(b + "ffn_gate.weight", cfg.ff, e)
            mat(b + "ffn_up.weight", cfg.ff, e)
            mat(b + "ffn_down.weight", e, cfg.ff)
            continue
        # the layer's head size, key/value heads, width and K/V source (Gemma 4, src/model.cpp:337-341)
        hdl, ffl = cfg.head_dim_of(l), cfg.ff_of(l)
        qdl, kvdl, own = cfg.heads * hdl, cfg.kv_heads_of(l) * hdl, cfg.kv_layer_of(l) == l
        if cfg.arch == ARCH_PHI3:  # fused Q|K|V and gate|up (src/model.cpp:370-380)
            mat(b + "attn_qkv.weight", qd + 2 * kvd, e)
        else:  # Qwen3.5: each head's query rows followed by its gate rows (src/model.cpp:383-384)
            mat(b + "attn_q.weight", 2 * qdl if cfg.arch == ARCH_QWEN35 else qdl, e)
            if own:
                mat(b + "attn_k.weight", kvdl, e)
                if cfg.arch != ARCH_GEMMA4 or f.tensor(b + "attn_v.weight") is not None:  # Gemma 4: K may serve as V
                    mat(b + "attn_v.weight", kvdl, e)
        if cfg.arch in (ARCH_QWEN3, ARCH_GEMMA3, ARCH_LFM2, ARCH_QWEN35, ARCH_GEMMA4):
            vec(b + "attn_q_norm.weight", hdl)
            if own:
                vec(b + "attn_k_norm.weight", hdl)
        if cfg.arch in (ARCH_GEMMA3, ARCH_GEMMA4):
            vec(b + "post_attention_norm.weight", e)
            vec(b + "post_ffw_norm.weight", e)
        if cfg.arch == ARCH_BITNET:
            vec(b + "attn_sub_norm.weight", e)
            vec(b + "ffn_sub_norm.weight", cfg.ff)
        if cfg.ple_dim:  # src/model.cpp:403-407
            mat(b + "inp_gate.weight", cfg.ple_dim, e)
            mat(b + "proj.weight", e, cfg.ple_dim)
            vec(b + "post_norm.weight", e)
        if f.tensor(b + "layer_output_scale.weight") is not None:  # src/model.cpp:408-410
            vec(b + "layer_output_scale.weight", 1)
        if f.tensor(b + "attn_q.bias") is not None:  # all or none (src/model.cpp:411-416)
            vec(b + "attn_q.bias", qd)
            vec(b + "attn_k.bias", kvd)
            vec(b + "attn_v.bias", kvd)
        mat(b + "attn_output.weight", e, qdl)
        vec(b + ("post_attention_norm.weight" if cfg.arch == ARCH_QWEN35 else "ffn_norm.weight"), e)  # src/model.cpp:418
        if cfg.arch == ARCH_PHI3:
            mat(b + "ffn_up.weight", 2 * cfg.ff, e)
        else:
            mat(b + "ffn_gate.weight", ffl, e)
            mat(b + "ffn_up.weight", ffl, e)
        mat(b + "ffn_down.weight", e, ffl)
    return out


def load(path: str):
    """(GgufFile, ModelConfig, tensor table) of a model file."""
    f = G.GgufFile(path)
    cfg = parse_config(f)
    return f, cfg, tensor_table(f, cfg)
