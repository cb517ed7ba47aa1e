"""Seeded random-weight GGUF models of the benchmark shapes.

Every byte comes from a counter-based splitmix64 stream (integer arithmetic
only) and exact float64 operations, so a file is byte-identical on every
machine: the reference's CPU engine and the HIP session read the very same
weights here and on the GPU host.  Tensor names, shapes and metadata keys are
the ones the reference's loader reads (src/model.cpp:161-301, :303-423): GGUF
dims innermost first, so a rows x cols matrix is stored as {cols, rows}
(src/model.cpp:462).

Distributions (where a config leaves a scale open it is
pinned here so activations stay O(1) through the layers):
  Q4_0  d = half(U(0.001, 0.02)), nibbles uniform 0..15
  Q8_0  d = half(U(0.0002, 0.004)), values uniform -127..127
  Q4_K  d, dmin = half(U(0.0001, 0.001)), 6-bit scales/mins and nibbles uniform
  Q6_K  d = half(U(0.00002, 0.0002)), int8 sub-block scales uniform -32..31, 6-bit values uniform
  TQ2_0 codes uniform over {0, 1, 2} (weights -1, 0, 1), one fp16 scale per tensor U(0.01, 0.03)
  norm weights f32 U(0.8, 1.2)
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

import numpy as np

from . import gguf as G

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 started at ``seed`` (counter form: output i mixes seed + (i+1)*golden)."""
    with np.errstate(over="ignore"):
        z = np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN + np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for b in text.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def stream_seed(model_seed: int, name: str) -> int:
    return (fnv1a64(name) ^ (model_seed * 0xD1B54A32D192ED03)) & 0xFFFFFFFFFFFFFFFF


def random_bytes(seed: int, n: int) -> np.ndarray:
    return splitmix64(seed, (n + 7) // 8).view(np.uint8)[:n]


def random_unit(seed: int, n: int) -> np.ndarray:
    """Uniform [0, 1) float64 with 53 random bits (exact)."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def random_uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    return lo + random_unit(seed, n) * (hi - lo)


def random_normalish(seed: int, n: int) -> np.ndarray:
    """Approximately N(0, 1): Irwin-Hall sum of four uniforms, centred and scaled (exact float64 ops only)."""
    u = random_unit(seed, 4 * n).reshape(n, 4)
    return (u.sum(axis=1) - 2.0) * 1.7320508075688772


def half_bits(x: np.ndarray) -> np.ndarray:
    """float64 -> float32 -> IEEE half (round to nearest even) as uint16."""
    return x.astype(np.float32).astype(np.float16).view(np.uint16)


# --------------------------------------------------------------------------- blocks

def q4_0_blocks(seed: int, nblocks: int) -> np.ndarray:
    out = np.empty((nblocks, 18), np.uint8)
    out[:, 0:2] = half_bits(random_uniform(seed, nblocks, 0.001, 0.02)).view(np.uint8).reshape(nblocks, 2)
    out[:, 2:18] = random_bytes(seed ^ 0x5151, nblocks * 16).reshape(nblocks, 16)
    return out


def q8_0_blocks(seed: int, nblocks: int, lo=0.0002, hi=0.004) -> np.ndarray:
    out = np.empty((nblocks, 34), np.uint8)
    out[:, 0:2] = half_bits(random_uniform(seed, nblocks, lo, hi)).view(np.uint8).reshape(nblocks, 2)
    raw = random_bytes(seed ^ 0x5252, nblocks * 32).astype(np.int16)
    out[:, 2:34] = ((raw % 255) - 127).astype(np.int8).view(np.uint8).reshape(nblocks, 32)
    return out


def q4_k_blocks(seed: int, nblocks: int) -> np.ndarray:
    out = np.empty((nblocks, 144), np.uint8)
    out[:, 0:2] = half_bits(random_uniform(seed, nblocks, 0.0001, 0.001)).view(np.uint8).reshape(nblocks, 2)
    out[:, 2:4] = half_bits(random_uniform(seed ^ 0x1, nblocks, 0.0001, 0.001)).view(np.uint8).reshape(nblocks, 2)
    out[:, 4:144] = random_bytes(seed ^ 0x5353, nblocks * 140).reshape(nblocks, 140)
    return out


def q6_k_blocks(seed: int, nblocks: int) -> np.ndarray:
    out = np.empty((nblocks, 210), np.uint8)
    out[:, 0:192] = random_bytes(seed ^ 0x5454, nblocks * 192).reshape(nblocks, 192)       # ql, qh
    sc = (random_bytes(seed ^ 0x5555, nblocks * 16).astype(np.int16) % 64) - 32
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8).reshape(nblocks, 16)
    out[:, 208:210] = half_bits(random_uniform(seed, nblocks, 0.00002, 0.0002)).view(np.uint8).reshape(nblocks, 2)
    return out


def tq2_0_blocks(seed: int, nblocks: int) -> np.ndarray:
    out = np.empty((nblocks, 66), np.uint8)
    codes = (splitmix64(seed ^ 0x5656, nblocks * 256) % np.uint64(3)).astype(np.uint8).reshape(nblocks, 4, 64)
    # byte m of the 64 holds elements in bit pairs 2l (src/quant.h:123-130): we only need uniform
    # codes, so pack four independent codes per byte.
    packed = codes[:, 0] | (codes[:, 1] << 2) | (codes[:, 2] << 4) | (codes[:, 3] << 6)
    out[:, 0:64] = packed
    d = half_bits(random_uniform(seed ^ 0x77, 1, 0.01, 0.03))  # one scale per tensor
    out[:, 64:66] = np.broadcast_to(d.view(np.uint8), (nblocks, 2))
    return out


def q4_1_blocks(seed: int, nblocks: int) -> np.ndarray:
    """{d, m, qs[16]}: d ~ U(0.001, 0.02), m ~ U(-0.15, 0) so that q d + m centres near zero."""
    out = np.empty((nblocks, 20), np.uint8)
    out[:, 0:2] = half_bits(random_uniform(seed, nblocks, 0.001, 0.02)).view(np.uint8).reshape(nblocks, 2)
    out[:, 2:4] = half_bits(random_uniform(seed ^ 0x2, nblocks, -0.15, 0.0)).view(np.uint8).reshape(nblocks, 2)
    out[:, 4:20] = random_bytes(seed ^ 0x5757, nblocks * 16).reshape(nblocks, 16)
    return out


def q5_0_blocks(seed: int, nblocks: int) -> np.ndarray:
    """{d, qh[4], qs[16]}: d ~ U(0.001, 0.02), the 5-bit values uniform."""
    out = np.empty((nblocks, 22), np.uint8)
    out[:, 0:2] = half_bits(random_uniform(seed, nblocks, 0.001, 0.02)).view(np.uint8).reshape(nblocks, 2)
    out[:, 2:22] = random_bytes(seed ^ 0x5858, nblocks * 20).reshape(nblocks, 20)
    return out


def q5_k_blocks(seed: int, nblocks: int) -> np.ndarray:
    """{d, dmin, scales[12], qh[32], qs[128]}: d, dmin ~ U(0.0001, 0.001), scales and values uniform."""
    out = np.empty((nblocks, 176), np.uint8)
    out[:, 0:2] = half_bits(random_uniform(seed, nblocks, 0.0001, 0.001)).view(np.uint8).reshape(nblocks, 2)
    out[:, 2:4] = half_bits(random_uniform(seed ^ 0x1, nblocks, 0.0001, 0.001)).view(np.uint8).reshape(nblocks, 2)
    out[:, 4:176] = random_bytes(seed ^ 0x5959, nblocks * 172).reshape(nblocks, 172)
    return out


BLOCK_MAKERS = {G.T_Q4_0: q4_0_blocks, G.T_Q8_0: q8_0_blocks, G.T_Q4_K: q4_k_blocks,
                G.T_Q6_K: q6_k_blocks, G.T_TQ2_0: tq2_0_blocks,
                G.T_Q4_1: q4_1_blocks, G.T_Q5_0: q5_0_blocks, G.T_Q5_K: q5_k_blocks}


# --------------------------------------------------------------------------- models

@dataclass
class ModelSpec:
    name: str
    arch: str                 # general.architecture
    embd: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    ff: int
    vocab: int
    rope_base: float
    eps: float = 1e-6
    context: int = 40960
    fmt: dict = field(default_factory=dict)   # role -> tensor type; roles: q k v o gate up down
    embd_fmt: int = G.T_Q8_0
    out_fmt: int | None = G.T_Q8_0            # None: tied to token_embd (src/model.cpp:328-330)
    seed: int = 1
    extra: dict = field(default_factory=dict)  # further "<arch>.<key>" metadata: key -> (GGUF type, value)
    factors: dict = field(default_factory=dict)  # RoPE factor tensors: name -> length
    conv_layers: tuple = ()                      # LFM2: layers that convolve (head_count_kv entry 0)
    recurrent_layers: tuple = ()                 # Qwen3.5: Gated DeltaNet layers (all but every interval-th)
    no_v_layers: tuple = ()                      # Gemma 4: layers without attn_v (K serves as V)

    @property
    def query_dim(self):
        return self.heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim

    def layer_weight_bytes(self) -> int:
        """Quantised bytes of one layer's seven matrices."""
        shapes = {"q": (self.query_dim, self.embd), "k": (self.kv_dim, self.embd), "v": (self.kv_dim, self.embd),
                  "o": (self.embd, self.query_dim), "gate": (self.ff, self.embd), "up": (self.ff, self.embd),
                  "down": (self.embd, self.ff)}
        total = 0
        for role, (r, c) in shapes.items():
            be, bb = G.BLOCK[self.fmt[role]]
            total += r * c // be * bb
        return total

    def output_bytes(self) -> int:
        t = self.out_fmt if self.out_fmt is not None else self.embd_fmt
        be, bb = G.BLOCK[t]
        return self.vocab * self.embd // be * bb

    def decode_bytes(self, position: int) -> int:
        """Algorithmic HBM bytes of one decode step at context length ``position`` (weights + norms + KV)."""
        be, bb = G.BLOCK[self.embd_fmt]
        norms = 4 * (2 * self.embd + (2 * self.head_dim if self.arch == "qwen3" else 0)) * self.layers + 4 * self.embd
        if self.arch.startswith("bitnet"):
            norms += 4 * (self.embd + self.ff) * self.layers
        kv = 2 * 2 * self.kv_dim * self.layers * (position + 1)
        return self.layers * self.layer_weight_bytes() + self.output_bytes() + self.embd // be * bb + norms + kv


def _uniform4(t):
    return {r: t for r in ("q", "k", "v", "o", "gate", "up", "down")}


SPECS = {
    # Qwen3-0.6B shape, Q4_0 layers, Q8_0 embeddings and output.
    "qwen3-0.6b": ModelSpec("qwen3-0.6b", "qwen3", 1024, 28, 16, 8, 128, 3072, 151936, 1e6, fmt=_uniform4(G.T_Q4_0)),
    # Llama-3.2-1B shape in a Q4_K_M mix; tied Q6_K embedding.
    "llama-3.2-1b": ModelSpec("llama-3.2-1b", "llama", 2048, 16, 32, 8, 64, 8192, 128256, 5e5, eps=1e-5, context=131072,
                              fmt={**_uniform4(G.T_Q4_K), "v": G.T_Q6_K, "down": G.T_Q6_K},
                              embd_fmt=G.T_Q6_K, out_fmt=None),
    # Qwen3-1.7B shape, all Q8_0.
    "qwen3-1.7b": ModelSpec("qwen3-1.7b", "qwen3", 2048, 28, 16, 8, 128, 6144, 151936, 1e6, fmt=_uniform4(G.T_Q8_0)),
    # BitNet b1.58 2B4T shape, TQ2_0 layers; tied Q4_0 embedding.
    "bitnet-2b": ModelSpec("bitnet-2b", "bitnet-b1.58", 2560, 30, 20, 5, 128, 6912, 128256, 5e5, eps=1e-5, context=4096,
                           fmt=_uniform4(G.T_TQ2_0), embd_fmt=G.T_Q4_0, out_fmt=None),
    # Small shapes of each family for the parity tests (the oracle finishes them in well under a second).
    "tiny-qwen3": ModelSpec("tiny-qwen3", "qwen3", 256, 2, 4, 2, 64, 512, 1000, 1e6, context=1024, fmt=_uniform4(G.T_Q4_0)),
    # tiny-qwen3's shape with a 16384-position context, for long pre-filled caches
    "tiny-qwen3-long": ModelSpec("tiny-qwen3-long", "qwen3", 256, 2, 4, 2, 64, 512, 1000, 1e6, context=16384,
                                 fmt=_uniform4(G.T_Q4_0)),
    "tiny-llama": ModelSpec("tiny-llama", "llama", 512, 2, 8, 2, 64, 768, 1000, 5e5, eps=1e-5, context=1024,
                            fmt={**_uniform4(G.T_Q4_K), "v": G.T_Q6_K, "down": G.T_Q6_K}, embd_fmt=G.T_Q6_K, out_fmt=None),
    # Feed-forward rows wider than the GEMV's activation buffer (8192): 4B-class widths.
    "tiny-wide": ModelSpec("tiny-wide", "llama", 256, 2, 4, 2, 64, 9728, 1000, 5e5, eps=1e-5, context=1024,
                           fmt={**_uniform4(G.T_Q4_K), "v": G.T_Q6_K, "down": G.T_Q6_K}, embd_fmt=G.T_Q6_K, out_fmt=None),
    "tiny-wide-q4": ModelSpec("tiny-wide-q4", "qwen3", 256, 2, 4, 2, 64, 14336, 1000, 1e6, context=1024,
                              fmt=_uniform4(G.T_Q4_0)),
    "tiny-q8": ModelSpec("tiny-q8", "qwen3", 256, 2, 4, 2, 64, 512, 1000, 1e6, context=1024, fmt=_uniform4(G.T_Q8_0)),
    "tiny-bitnet": ModelSpec("tiny-bitnet", "bitnet-b1.58", 512, 2, 4, 1, 128, 768, 1000, 5e5, eps=1e-5, context=1024,
                             fmt=_uniform4(G.T_TQ2_0), embd_fmt=G.T_Q4_0, out_fmt=None),
    # The loader's other formats (a Q5_K_M mix; Q5_0 with Q4_1), on the path's families.
    "tiny-q5k": ModelSpec("tiny-q5k", "llama", 512, 2, 8, 2, 64, 768, 1000, 5e5, eps=1e-5, context=1024,
                          fmt={**_uniform4(G.T_Q5_K), "v": G.T_Q6_K, "down": G.T_Q6_K}, embd_fmt=G.T_Q6_K, out_fmt=None),
    # Qwen2 (projection biases, no Q/K norms) and SmolLM3 (Llama-shaped, layers 3 and 7 without RoPE).
    "tiny-qwen2": ModelSpec("tiny-qwen2", "qwen2", 256, 2, 4, 2, 64, 512, 1000, 1e6, context=1024, fmt=_uniform4(G.T_Q4_0)),
    "tiny-smollm3": ModelSpec("tiny-smollm3", "smollm3", 512, 8, 8, 2, 64, 768, 1000, 5e5, eps=1e-5, context=1024,
                              fmt={**_uniform4(G.T_Q4_K), "v": G.T_Q6_K, "down": G.T_Q6_K}, embd_fmt=G.T_Q6_K, out_fmt=None),
    # Gemma 3: layers 0-4 and 6 slide over the last 8 positions (local RoPE base), 5 is global with
    # positions scaled by 1/2; logits soft-capped at 30; the Q8_0 embedding rows scaled by sqrt(embd).
    # Rows of 32-value blocks that end inside a 256-value chunk (Gemma-3-1B's 1152): 352 = 11 blocks,
    # 1184 = 37 blocks, so the batched GEMMs' last chunk holds 3 and 5 blocks.
    "tiny-gemma3w": ModelSpec("tiny-gemma3w", "gemma3", 352, 3, 4, 1, 64, 1184, 1000, 1e6, context=1024,
                              fmt=_uniform4(G.T_Q4_0),
                              extra={"attention.sliding_window": (G.U32, 8), "rope.freq_base_swa": (G.F32, 10000.0),
                                     "final_logit_softcapping": (G.F32, 30.0)}),
    "tiny-q8w": ModelSpec("tiny-q8w", "qwen3", 352, 2, 4, 2, 64, 1184, 1000, 1e6, context=1024, fmt=_uniform4(G.T_Q8_0)),
    "tiny-gemma3": ModelSpec("tiny-gemma3", "gemma3", 256, 7, 4, 1, 64, 512, 1000, 1e6, context=1024,
                             fmt=_uniform4(G.T_Q8_0),
                             extra={"attention.sliding_window": (G.U32, 8), "rope.freq_base_swa": (G.F32, 10000.0),
                                    "rope.scaling.factor": (G.F32, 2.0), "final_logit_softcapping": (G.F32, 30.0)}),
    # Phi-3: fused tensors, 32 of 64 head dimensions rotated, LongRoPE short factors up to a
    # 512-position context and long ones past it, cos/sin times 1.19.
    "tiny-phi3": ModelSpec("tiny-phi3", "phi3", 256, 2, 4, 4, 64, 512, 1000, 1e4, eps=1e-5, context=2048,
                           fmt=_uniform4(G.T_Q4_0),
                           extra={"rope.dimension_count": (G.U32, 32), "rope.scaling.attn_factor": (G.F32, 1.1902381),
                                  "rope.scaling.original_context_length": (G.U32, 512)},
                           factors={"rope_factors_short.weight": 16, "rope_factors_long.weight": 16}),
    # Llama 3.x's rope_freqs factors (src/model.cpp:314-318) on the tiny Llama shape.
    "tiny-llama32": ModelSpec("tiny-llama32", "llama", 512, 2, 8, 2, 64, 768, 1000, 5e5, eps=1e-5, context=1024,
                              fmt={**_uniform4(G.T_Q4_K), "v": G.T_Q6_K, "down": G.T_Q6_K}, embd_fmt=G.T_Q6_K,
                              out_fmt=None, factors={"rope_freqs.weight": 32}),
    # LFM2: layers 0, 1 and 3 are 3-tap short convolutions, layer 2 attends.
    "tiny-lfm2": ModelSpec("tiny-lfm2", "lfm2", 256, 4, 4, 2, 64, 512, 1000, 1e6, eps=1e-5, context=1024,
                           fmt=_uniform4(G.T_Q8_0), conv_layers=(0, 1, 3),
                           extra={"shortconv.l_cache": (G.U32, 3),
                                  "attention.head_count_kv": (G.ARRAY, (G.U32, [0, 0, 2, 0]))}),
    # Qwen3.5: layers 0, 1, 3 and 4 are Gated DeltaNet recurrences (4 heads of a 64 x 64 state, 4-tap
    # conv), layers 2 and 5 attend with a sigmoid gate per query row and 16 of 64 head dimensions
    # rotated; head 1's dt bias of 20 puts its softplus on both sides of the reference's cut-over.
    "tiny-qwen35": ModelSpec("tiny-qwen35", "qwen35", 256, 6, 4, 2, 64, 512, 1000, 1e7, context=1024,
                             fmt=_uniform4(G.T_Q8_0), recurrent_layers=(0, 1, 3, 4),
                             extra={"full_attention_interval": (G.U32, 3), "rope.dimension_count": (G.U32, 16),
                                    "ssm.state_size": (G.U32, 64), "ssm.group_count": (G.U32, 4),
                                    "ssm.time_step_rank": (G.U32, 4), "ssm.inner_size": (G.U32, 256),
                                    "ssm.conv_kernel": (G.U32, 4)}),
    # The same family at a 128 x 128 state and head size, Q4_0 layers, a 3-tap conv.
    "tiny-qwen35w": ModelSpec("tiny-qwen35w", "qwen35", 512, 4, 4, 1, 128, 768, 1000, 1e7, context=1024,
                              fmt=_uniform4(G.T_Q4_0), recurrent_layers=(0, 1, 2),
                              extra={"full_attention_interval": (G.U32, 4), "rope.dimension_count": (G.U32, 32),
                                     "ssm.state_size": (G.U32, 128), "ssm.group_count": (G.U32, 4),
                                     "ssm.time_step_rank": (G.U32, 4), "ssm.inner_size": (G.U32, 512),
                                     "ssm.conv_kernel": (G.U32, 3)}),
    # Qwen3.5's own attention shape: 256-wide heads with a quarter of each rotated (the plain attention).
    "tiny-qwen35h": ModelSpec("tiny-qwen35h", "qwen35", 256, 4, 4, 2, 256, 512, 1000, 1e7, context=1024,
                              fmt=_uniform4(G.T_Q8_0), recurrent_layers=(0, 1, 2),
                              extra={"full_attention_interval": (G.U32, 4), "rope.dimension_count": (G.U32, 64),
                                     "ssm.state_size": (G.U32, 64), "ssm.group_count": (G.U32, 4),
                                     "ssm.time_step_rank": (G.U32, 4), "ssm.inner_size": (G.U32, 256),
                                     "ssm.conv_kernel": (G.U32, 4)}),
    # Gemma 4: sliding layers 0-2 and 4 (64-wide heads, 2 key/value heads) and global layers 3 and 5
    # (128-wide heads, 1 key/value head, proportional RoPE factors); layers 4 and 5 read the caches
    # of layers 2 and 3; layer 3 has no V projection (K serves as V); per-layer feed-forward widths,
    # 256-wide per-layer embeddings and per-layer output scales.
    "tiny-gemma4": ModelSpec("tiny-gemma4", "gemma4", 256, 6, 4, 2, 128, 768, 1000, 1e6, context=1024,
                             fmt=_uniform4(G.T_Q8_0), factors={"rope_freqs.weight": 64}, no_v_layers=(3,),
                             extra={"attention.sliding_window": (G.U32, 8), "rope.freq_base_swa": (G.F32, 10000.0),
                                    "final_logit_softcapping": (G.F32, 30.0),
                                    "attention.sliding_window_pattern": (G.ARRAY, (G.BOOL, [1, 1, 1, 0, 1, 0])),
                                    "attention.key_length_swa": (G.U32, 64),
                                    "attention.shared_kv_layers": (G.U32, 2),
                                    "embedding_length_per_layer_input": (G.U32, 256),
                                    "feed_forward_length": (G.ARRAY, (G.I32, [512, 512, 768, 768, 512, 512])),
                                    "attention.head_count_kv": (G.ARRAY, (G.U32, [2, 2, 2, 1, 2, 1]))}),
    # Full-size shapes of the graph-path families, for bench.py's decode lines (synthetic weights):
    # Gemma-3-1B (256-wide heads: the plain attention; 512-position windows, five of six layers),
    # LFM2-1.2B (10 convolution layers, 6 attention layers), a Qwen3.5 shape (18 recurrent layers of
    # 16 128-wide heads, 6 attention layers of 256-wide heads) and a Gemma 4 shape (256/512-wide
    # heads, 15 shared K/V layers, 256-wide per-layer embeddings; its vocabulary cut to 65536 to
    # bound the per-layer table's size).
    "gemma3-1b": ModelSpec("gemma3-1b", "gemma3", 1152, 26, 4, 1, 256, 6912, 262144, 1e6, context=32768,
                           fmt=_uniform4(G.T_Q4_0),
                           extra={"attention.sliding_window": (G.U32, 512), "rope.freq_base_swa": (G.F32, 10000.0)}),
    "lfm2-1.2b": ModelSpec("lfm2-1.2b", "lfm2", 2048, 16, 32, 8, 64, 8192, 65536, 1e6, eps=1e-5, context=32768,
                           fmt=_uniform4(G.T_Q4_0), conv_layers=(0, 1, 3, 4, 6, 7, 9, 11, 13, 15),
                           extra={"shortconv.l_cache": (G.U32, 3),
                                  "attention.head_count_kv": (G.ARRAY, (G.U32, [0 if l in (0, 1, 3, 4, 6, 7, 9, 11, 13, 15)
                                                                                else 8 for l in range(16)]))}),
    "qwen35-0.8b": ModelSpec("qwen35-0.8b", "qwen35", 1024, 24, 8, 2, 256, 3584, 151936, 1e7, context=32768,
                             fmt=_uniform4(G.T_Q4_0), recurrent_layers=tuple(l for l in range(24) if (l + 1) % 4),
                             extra={"full_attention_interval": (G.U32, 4), "rope.dimension_count": (G.U32, 64),
                                    "ssm.state_size": (G.U32, 128), "ssm.group_count": (G.U32, 16),
                                    "ssm.time_step_rank": (G.U32, 16), "ssm.inner_size": (G.U32, 2048),
                                    "ssm.conv_kernel": (G.U32, 4)}),
    "gemma4-e2b": ModelSpec("gemma4-e2b", "gemma4", 1536, 35, 8, 1, 512, 6144, 65536, 1e6, context=32768,
                            fmt=_uniform4(G.T_Q4_0), embd_fmt=G.T_Q4_0,
                            extra={"attention.sliding_window": (G.U32, 512), "rope.freq_base_swa": (G.F32, 10000.0),
                                   "final_logit_softcapping": (G.F32, 30.0),
                                   "attention.sliding_window_pattern": (G.ARRAY, (G.BOOL, [0 if l % 5 == 4 else 1
                                                                                          for l in range(35)])),
                                   "attention.key_length_swa": (G.U32, 256),
                                   "attention.shared_kv_layers": (G.U32, 15),
                                   "embedding_length_per_layer_input": (G.U32, 256)}),
    "tiny-q5": ModelSpec("tiny-q5", "qwen3", 256, 2, 4, 2, 64, 512, 1000, 1e6, context=1024,
                         fmt={**_uniform4(G.T_Q5_0), "o": G.T_Q4_1, "down": G.T_Q4_1}),
}


def _matrix(w: G.GgufWriter, spec: ModelSpec, name: str, rows: int, cols: int, ttype: int):
    be, _ = G.BLOCK[ttype]
    nblocks = rows * cols // be
    seed = stream_seed(spec.seed, name)
    w.add_tensor(name, (cols, rows), ttype, lambda: BLOCK_MAKERS[ttype](seed, nblocks))


def _vector(w: G.GgufWriter, spec: ModelSpec, name: str, n: int):
    seed = stream_seed(spec.seed, name)
    w.add_tensor(name, (n,), G.T_F32, lambda: random_uniform(seed, n, 0.8, 1.2).astype(np.float32).view(np.uint8))


def _bias(w: G.GgufWriter, spec: ModelSpec, name: str, n: int):
    seed = stream_seed(spec.seed, name)
    w.add_tensor(name, (n,), G.T_F32, lambda: random_uniform(seed, n, -1.0, 1.0).astype(np.float32).view(np.uint8))


class _Gemma4Layers:
    """Per-layer shapes of a Gemma 4 spec, from its metadata (ModelConfig's accessors, src/model.h:87-118)."""

    def __init__(self, spec: ModelSpec):
        ex = spec.extra
        self.spec = spec
        self.pattern = list(ex["attention.sliding_window_pattern"][1][1])
        self.hd_local = ex.get("attention.key_length_swa", (None, 0))[1]
        self.shared = ex.get("attention.shared_kv_layers", (None, 0))[1]
        self.ple = ex.get("embedding_length_per_layer_input", (None, 0))[1]
        self.ffs = list(ex["feed_forward_length"][1][1]) if "feed_forward_length" in ex else [spec.ff] * spec.layers
        self.kvs = list(ex["attention.head_count_kv"][1][1]) if "attention.head_count_kv" in ex else [spec.kv_heads] * spec.layers

    def head_dim(self, l):
        return self.hd_local if self.hd_local and self.pattern[l] else self.spec.head_dim

    def kv(self, l):
        return self.kvs[l]

    def ff(self, l):
        return self.ffs[l]

    def kv_layer(self, l):
        start = self.spec.layers - self.shared if self.shared else 0
        if start == 0 or l < start:
            return l
        return start - (2 if self.pattern[l] else 1)


def write_model(spec: ModelSpec, path: str) -> str:
    """Writes ``spec`` as a GGUF file at ``path`` (skipped when the file already exists)."""
    if os.path.exists(path):
        return path
    a = spec.arch
    w = G.GgufWriter()
    w.add("general.architecture", G.STRING, a)
    w.add("general.name", G.STRING, f"brisk-synthetic-{spec.name}")
    w.add(f"{a}.embedding_length", G.U32, spec.embd)
    w.add(f"{a}.block_count", G.U32, spec.layers)
    w.add(f"{a}.attention.head_count", G.U32, spec.heads)
    if "attention.head_count_kv" not in spec.extra:
        w.add(f"{a}.attention.head_count_kv", G.U32, spec.kv_heads)
    w.add(f"{a}.attention.key_length", G.U32, spec.head_dim)
    w.add(f"{a}.attention.value_length", G.U32, spec.head_dim)
    if "feed_forward_length" not in spec.extra:
        w.add(f"{a}.feed_forward_length", G.U32, spec.ff)
    w.add(f"{a}.context_length", G.U32, spec.context)
    w.add(f"{a}.rope.freq_base", G.F32, spec.rope_base)
    w.add(f"{a}.attention.layer_norm_rms_epsilon", G.F32, spec.eps)
    for key, (vtype, value) in spec.extra.items():
        w.add(f"{a}.{key}", vtype, value)
    _matrix(w, spec, "token_embd.weight", spec.vocab, spec.embd, spec.embd_fmt)
    for name, n in spec.factors.items():  # per-frequency RoPE factors in [1, 8], as Llama 3's and LongRoPE's
        seed = stream_seed(spec.seed, name)
        w.add_tensor(name, (n,), G.T_F32, lambda seed=seed, n=n: random_uniform(seed, n, 1.0, 8.0).astype(np.float32).view(np.uint8))
    _vector(w, spec, "token_embd_norm.weight" if a == "lfm2" else "output_norm.weight", spec.embd)
    g4 = _Gemma4Layers(spec) if a == "gemma4" else None
    if g4 is not None and g4.ple:  # per-layer embeddings (src/model.cpp:319-324)
        _matrix(w, spec, "per_layer_token_embd.weight", spec.vocab, g4.ple * spec.layers, spec.embd_fmt)
        _matrix(w, spec, "per_layer_model_proj.weight", g4.ple * spec.layers, spec.embd, spec.fmt["q"])
        _vector(w, spec, "per_layer_proj_norm.weight", g4.ple)
    if spec.out_fmt is not None:
        _matrix(w, spec, "output.weight", spec.vocab, spec.embd, spec.out_fmt)
    for l in range(spec.layers):
        b = f"blk.{l}."
        _vector(w, spec, b + "attn_norm.weight", spec.embd)
        if l in spec.recurrent_layers:  # Qwen3.5 Gated DeltaNet (src/model.cpp:343-358)
            ex = spec.extra
            state, heads, inner, taps = (ex[k][1] for k in ("ssm.state_size", "ssm.time_step_rank", "ssm.inner_size",
                                                            "ssm.conv_kernel"))
            qkv = 2 * ex["ssm.group_count"][1] * state + inner
            _matrix(w, spec, b + "attn_qkv.weight", qkv, spec.embd, spec.fmt["q"])
            _matrix(w, spec, b + "attn_gate.weight", inner, spec.embd, spec.fmt["q"])
            _matrix(w, spec, b + "ssm_alpha.weight", heads, spec.embd, spec.fmt["k"])
            _matrix(w, spec, b + "ssm_beta.weight", heads, spec.embd, spec.fmt["k"])
            seed = stream_seed(spec.seed, b + "ssm_a")  # A = -exp(A_log) < 0: every decay below 1
            w.add_tensor(b + "ssm_a", (heads,), G.T_F32,
                         lambda seed=seed, n=heads: random_uniform(seed, n, -4.0, -0.5).astype(np.float32).view(np.uint8))
            seed = stream_seed(spec.seed, b + "ssm_dt")
            dt = random_uniform(seed, heads, -1.0, 1.0)
            dt[1] = 20.0
            w.add_tensor(b + "ssm_dt.bias", (heads,), G.T_F32, lambda dt=dt: dt.astype(np.float32).view(np.uint8))
            seed = stream_seed(spec.seed, b + "ssm_conv1d")
            w.add_tensor(b + "ssm_conv1d.weight", (taps, qkv), G.T_F32,
                         lambda seed=seed, n=taps * qkv: random_uniform(seed, n, -1.0, 1.0).astype(np.float32).view(np.uint8))
            _vector(w, spec, b + "ssm_norm.weight", state)
            _matrix(w, spec, b + "ssm_out.weight", spec.embd, inner, spec.fmt["o"])
            _vector(w, spec, b + "post_attention_norm.weight", spec.embd)
            _matrix(w, spec, b + "ffn_gate.weight", spec.ff, spec.embd, spec.fmt["gate"])
            _matrix(w, spec, b + "ffn_up.weight", spec.ff, spec.embd, spec.fmt["up"])
            _matrix(w, spec, b + "ffn_down.weight", spec.embd, spec.ff, spec.fmt["down"])
            continue
        if l in spec.conv_layers:  # LFM2 short convolution (src/model.cpp:360-364)
            taps = spec.extra["shortconv.l_cache"][1]
            _matrix(w, spec, b + "shortconv.in_proj.weight", 3 * spec.embd, spec.embd, spec.fmt["q"])
            _matrix(w, spec, b + "shortconv.out_proj.weight", spec.embd, spec.embd, spec.fmt["o"])
            seed = stream_seed(spec.seed, b + "conv")
            w.add_tensor(b + "shortconv.conv.weight", (taps, spec.embd), G.T_F32,
                         lambda seed=seed, n=taps * spec.embd: random_uniform(seed, n, -1.0, 1.0).astype(np.float32).view(np.uint8))
            _vector(w, spec, b + "ffn_norm.weight", spec.embd)
            _matrix(w, spec, b + "ffn_gate.weight", spec.ff, spec.embd, spec.fmt["gate"])
            _matrix(w, spec, b + "ffn_up.weight", spec.ff, spec.embd, spec.fmt["up"])
            _matrix(w, spec, b + "ffn_down.weight", spec.embd, spec.ff, spec.fmt["down"])
            continue
        if g4 is not None:  # src/model.cpp:337-410
            hd, kvh, ff, own = g4.head_dim(l), g4.kv(l), g4.ff(l), g4.kv_layer(l) == l
            _matrix(w, spec, b + "attn_q.weight", spec.heads * hd, spec.embd, spec.fmt["q"])
            if own:
                _matrix(w, spec, b + "attn_k.weight", kvh * hd, spec.embd, spec.fmt["k"])
                if l not in spec.no_v_layers:  # else K serves as V (src/model.cpp:386-388)
                    _matrix(w, spec, b + "attn_v.weight", kvh * hd, spec.embd, spec.fmt["v"])
            _vector(w, spec, b + "attn_q_norm.weight", hd)
            if own:
                _vector(w, spec, b + "attn_k_norm.weight", hd)
            _vector(w, spec, b + "post_attention_norm.weight", spec.embd)
            _vector(w, spec, b + "post_ffw_norm.weight", spec.embd)
            if g4.ple:
                _matrix(w, spec, b + "inp_gate.weight", g4.ple, spec.embd, spec.fmt["gate"])
                _matrix(w, spec, b + "proj.weight", spec.embd, g4.ple, spec.fmt["down"])
                _vector(w, spec, b + "post_norm.weight", spec.embd)
            seed = stream_seed(spec.seed, b + "out_scale")
            w.add_tensor(b + "layer_output_scale.weight", (1,), G.T_F32,
                         lambda seed=seed: random_uniform(seed, 1, 0.5, 1.5).astype(np.float32).view(np.uint8))
            _matrix(w, spec, b + "attn_output.weight", spec.embd, spec.heads * hd, spec.fmt["o"])
            _vector(w, spec, b + "ffn_norm.weight", spec.embd)
            _matrix(w, spec, b + "ffn_gate.weight", ff, spec.embd, spec.fmt["gate"])
            _matrix(w, spec, b + "ffn_up.weight", ff, spec.embd, spec.fmt["up"])
            _matrix(w, spec, b + "ffn_down.weight", spec.embd, ff, spec.fmt["down"])
            continue
        if a == "phi3":  # fused Q|K|V (src/model.cpp:370-376)
            _matrix(w, spec, b + "attn_qkv.weight", spec.query_dim + 2 * spec.kv_dim, spec.embd, spec.fmt["q"])
        else:
            _matrix(w, spec, b + "attn_q.weight", (2 if a == "qwen35" else 1) * spec.query_dim, spec.embd, spec.fmt["q"])
            _matrix(w, spec, b + "attn_k.weight", spec.kv_dim, spec.embd, spec.fmt["k"])
            _matrix(w, spec, b + "attn_v.weight", spec.kv_dim, spec.embd, spec.fmt["v"])
        if a in ("qwen3", "gemma3", "lfm2", "qwen35"):
            _vector(w, spec, b + "attn_q_norm.weight", spec.head_dim)
            _vector(w, spec, b + "attn_k_norm.weight", spec.head_dim)
        if a == "gemma3":
            _vector(w, spec, b + "post_attention_norm.weight", spec.embd)
            _vector(w, spec, b + "post_ffw_norm.weight", spec.embd)
        if a.startswith("bitnet"):
            _vector(w, spec, b + "attn_sub_norm.weight", spec.embd)
            _vector(w, spec, b + "ffn_sub_norm.weight", spec.ff)
        if a == "qwen2":  # Q/K/V projection biases (src/model.cpp:411-416)
            _bias(w, spec, b + "attn_q.bias", spec.query_dim)
            _bias(w, spec, b + "attn_k.bias", spec.kv_dim)
            _bias(w, spec, b + "attn_v.bias", spec.kv_dim)
        _matrix(w, spec, b + "attn_output.weight", spec.embd, spec.query_dim, spec.fmt["o"])
        _vector(w, spec, b + ("post_attention_norm.weight" if a == "qwen35" else "ffn_norm.weight"), spec.embd)
        if a == "phi3":  # fused gate|up (src/model.cpp:377-379)
            _matrix(w, spec, b + "ffn_up.weight", 2 * spec.ff, spec.embd, spec.fmt["up"])
        else:
            _matrix(w, spec, b + "ffn_gate.weight", spec.ff, spec.embd, spec.fmt["gate"])
            _matrix(w, spec, b + "ffn_up.weight", spec.ff, spec.embd, spec.fmt["up"])
        _matrix(w, spec, b + "ffn_down.weight", spec.embd, spec.ff, spec.fmt["down"])
    tmp = path + ".part"
    w.write(tmp)
    os.replace(tmp, path)
    return path


def model_dir() -> str:
    d = os.environ.get("BRISK_MODEL_DIR") or os.path.join(os.environ.get("TMPDIR", "/tmp"), "brisk_models")
    os.makedirs(d, exist_ok=True)
    return d


def model_path(name: str) -> str:
    """Path of the seeded model ``name``, written on first use."""
    spec = SPECS[name]
    return write_model(spec, os.path.join(model_dir(), f"{name}-s{spec.seed}.gguf"))


def prompt_ids(n: int, vocab: int, seed: int = 7) -> np.ndarray:
    """``n`` seeded random token ids in [0, vocab)."""
    return (splitmix64(seed * 0x2545F4914F6CDD1D + 3, n) % np.uint64(vocab)).astype(np.int32)
