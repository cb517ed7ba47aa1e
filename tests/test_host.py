"""CPU tests of the host side — no GPU: the C-ABI library's exports, the GGUF
reader/writer, the model-config parser and the seeded synthetic models."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from brisk_hip import gguf as G, lib as hiplib, model, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "brisk_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(brisk_hip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    if not os.path.exists(hiplib.LIB_PATH):
        pytest.skip("libbrisk_hip.so is not built (run __graft_entry__.build())")
    so = C.CDLL(hiplib.LIB_PATH)
    names = declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing
    assert set(names) == set(hiplib.EXPORTS)


def test_library_host_only_calls():
    """Calls that touch no device: the ABI version and the packed-size arithmetic."""
    if not os.path.exists(hiplib.LIB_PATH):
        pytest.skip("libbrisk_hip.so is not built")
    L = hiplib.load()
    text = open(HEADER).read()
    want = int(re.search(r"#define BRISK_HIP_ABI_VERSION (\d+)", text).group(1))
    assert L.brisk_hip_abi_version() == want
    # packed planes hold exactly the GGUF bytes of the matrix, each plane 256-byte aligned
    for t, (be, bb) in ((G.T_Q4_0, (32, 18)), (G.T_Q8_0, (32, 34)), (G.T_Q4_K, (256, 144)), (G.T_Q6_K, (256, 210)),
                        (G.T_TQ2_0, (256, 66)), (G.T_Q4_1, (32, 20)), (G.T_Q5_0, (32, 22)), (G.T_Q5_K, (256, 176))):
        rows, cols = 48, 2048
        n = L.brisk_hip_packed_bytes(t, rows, cols)
        gguf = rows * cols // be * bb
        assert gguf <= n <= gguf + 3 * 256 + 64 * rows * cols // be
    assert L.brisk_hip_packed_bytes(G.T_Q4_0, 4, 33) == 0  # cols not a multiple of the block
    assert L.brisk_hip_packed_bytes(99, 4, 64) == 0


def test_gguf_round_trip(tmp_path):
    w = G.GgufWriter()
    w.add("general.architecture", G.STRING, "qwen3")
    w.add("qwen3.block_count", G.U32, 3)
    w.add("qwen3.rope.freq_base", G.F32, 1e6)
    w.add("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, ["a", "bc", "d"]))
    blocks = synth.q4_0_blocks(5, 8)
    w.add_tensor("blk.0.attn_q.weight", (64, 4), G.T_Q4_0, lambda: blocks)
    vec = np.arange(64, dtype=np.float32)
    w.add_tensor("output_norm.weight", (64,), G.T_F32, lambda: vec.view(np.uint8))
    path = str(tmp_path / "t.gguf")
    w.write(path)
    f = G.GgufFile(path)
    assert f.metadata["general.architecture"] == "qwen3"
    assert f.metadata["qwen3.block_count"] == 3
    assert f.metadata["tokenizer.ggml.tokens"] == ["a", "bc", "d"]
    t = f.tensors["blk.0.attn_q.weight"]
    assert t.type == G.T_Q4_0 and tuple(t.dims) == (64, 4)
    assert np.array_equal(np.asarray(t.data).reshape(-1), blocks.reshape(-1))
    assert np.array_equal(np.asarray(f.tensors["output_norm.weight"].data).view(np.float32), vec)


def test_gguf_rejects_bad_magic(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"XXXX" + b"\0" * 64)
    with pytest.raises(G.GgufError):
        G.GgufFile(str(p))


def test_synthetic_blocks_are_deterministic_and_in_range():
    a, b = synth.q4_0_blocks(9, 100), synth.q4_0_blocks(9, 100)
    assert np.array_equal(a, b)
    d = a[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all((d >= 0.0009) & (d <= 0.0201))  # configs[0]: d ~ U(0.001, 0.02)
    q8 = synth.q8_0_blocks(9, 100)
    assert np.all(q8[:, 2:].view(np.int8) >= -127)
    t = synth.tq2_0_blocks(9, 10)
    codes = np.stack([(t[:, :64] >> (2 * l)) & 3 for l in range(4)])
    assert codes.max() <= 2  # ternary codes 0..2 only


def test_spec_bytes_match_the_measurement_contract():
    """decode bytes of configs[1] (Qwen3-0.6B Q4_0 + Q8_0 output) at position 0."""
    s = synth.SPECS["qwen3-0.6b"]
    assert s.layers * s.layer_weight_bytes() == 247_726_080
    assert s.output_bytes() == 165_306_368


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama", "tiny-bitnet", "tiny-q5k", "tiny-q5", "tiny-qwen2", "tiny-smollm3", "tiny-gemma3", "tiny-phi3", "tiny-llama32", "tiny-lfm2"])
def test_model_config_parse(name):
    spec = synth.SPECS[name]
    f, cfg, table = model.load(synth.model_path(name))
    assert (cfg.embd, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.ff, cfg.vocab) == \
        (spec.embd, spec.layers, spec.heads, spec.kv_heads, spec.head_dim, spec.ff, spec.vocab)
    names = {t.name for t in table}
    assert "token_embd.weight" in names and "blk.0.ffn_down.weight" in names
    assert ("output.weight" in names) == (spec.out_fmt is not None)


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama", "tiny-bitnet", "tiny-q5k", "tiny-q5", "tiny-qwen2", "tiny-smollm3", "tiny-gemma3", "tiny-phi3", "tiny-llama32", "tiny-lfm2"])
def test_session_estimate(name):
    """brisk_hip_session_estimate (HBM counterpart of estimate_memory, src/memory.cpp:46-96): shapes only, no GPU."""
    from brisk_hip.session import estimate
    import brisk_hip
    lib = brisk_hip.load()
    f, cfg, table = model.load(synth.model_path(name))
    e1, e2 = estimate((f, cfg, table), 256), estimate((f, cfg, table), 512)
    kvd = cfg.kv_heads * cfg.head_dim
    # fp16 K and V for every position of an attention layer; an LFM2 short-convolution layer
    # (blk.N.shortconv.*) holds its bx rows instead (estimate_memory, src/memory.cpp:59-68)
    conv = sum(1 for t in table if t.name.endswith(".shortconv.in_proj.weight"))
    assert (conv > 0) == (name == "tiny-lfm2")
    assert e1["cache"] == 2 * (cfg.layers - conv) * kvd * 256 * 2 + conv * 256 * cfg.embd * 2
    assert e2["cache"] == 2 * e1["cache"]
    packed = sum(lib.brisk_hip_packed_bytes(t.type, t.rows, t.cols) for t in table if t.type != 0)
    vectors = sum(t.rows * t.cols * 4 for t in table if t.type == 0)
    assert e1["weights"] == packed + vectors
    assert e1["total"] == e1["weights"] + e1["cache"] + e1["scratch"]
    assert e2["scratch"] > e1["scratch"]  # the RoPE table and sequence grow with the context
    # max_context 0 is the model's own context length, and larger values are capped there
    assert estimate((f, cfg, table), 0) == estimate((f, cfg, table), 10 * cfg.context)


def test_header_structs_match_the_ctypes_binding(tmp_path):
    """sizeof and field offsets of include/brisk_hip.h's structs, compiled by the C compiler, equal the
    ctypes declarations (a caller built against another header version would pass another layout)."""
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("no C compiler")
    structs = {"brisk_hip_config": hiplib.HipConfig, "brisk_hip_tensor": hiplib.HipTensor, "brisk_hip_memory": hiplib.HipMemory}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "brisk_hip.h"', "int main(void) {"]
    for cname, ct in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in ct._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l.strip()}
    for cname, ct in structs.items():
        assert got[(cname, "size")] == C.sizeof(ct), cname
        for fname, _ in ct._fields_:
            assert got[(cname, fname)] == getattr(ct, fname).offset, (cname, fname)


def test_lfm2_layers_must_share_one_kv_head_count(tmp_path):
    """The session applies one key/value head count to every attention layer, so a model whose
    attention layers differ (head_count_kv per layer, src/model.cpp:229-238) is refused at load."""
    src = G.GgufFile(synth.model_path("tiny-lfm2"))
    kv = list(src.metadata["lfm2.attention.head_count_kv"])
    nz = [i for i, k in enumerate(kv) if k != 0]
    z = [i for i, k in enumerate(kv) if k == 0]
    assert nz and z
    kv[z[0]] = int(kv[nz[0]]) * 2  # a second attention layer with twice the key/value heads
    md = dict(src.metadata)
    md["lfm2.attention.head_count_kv"] = kv
    with pytest.raises(model.ModelError, match="different key/value head counts"):
        model.parse_config(_MetaOnly(md))


class _MetaOnly:
    """A GGUF stand-in carrying only metadata, for the config parser."""
    def __init__(self, metadata):
        self.metadata = metadata

    def get(self, key, default=None):
        return self.metadata.get(key, default)


def _mx_bytes(type_, rows, cols):
    """The expanded planes a batched prefill holds for one matrix: int8 lo and hi weights (rows padded
    to 128), float scales (Q4_K/Q5_K: d and dmin), and the K-quants' 8 sub-block mins a row."""
    align = lambda n: (n + 255) // 256 * 256  # noqa: E731
    rp, nsb = (rows + 127) // 128 * 128, cols // 256
    km = type_ in (G.T_Q4_K, G.T_Q5_K)
    return rp * cols * 2 + align(rp * nsb * (2 if km else 1) * 4) + (align(rp * nsb * 8) if km else 0)


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-q5k"])
def test_session_estimate_counts_expanded_planes(name, monkeypatch):
    """The estimate charges the prefill's expanded planes: switching Q4_K expansion on
    (BRISK_HIP_PREFILL_Q4X=1) adds exactly their bytes for every Q4_K layer matrix."""
    from brisk_hip.session import estimate
    f, cfg, table = model.load(synth.model_path(name))
    monkeypatch.delenv("BRISK_HIP_PREFILL_Q4X", raising=False)
    base = estimate((f, cfg, table), 256)
    monkeypatch.setenv("BRISK_HIP_PREFILL_Q4X", "1")
    more = estimate((f, cfg, table), 256)
    want = sum(_mx_bytes(t.type, t.rows, t.cols) for t in table if t.type == G.T_Q4_K and t.name.startswith("blk."))
    assert more["scratch"] - base["scratch"] == want
    assert (want > 0) == (name == "tiny-llama")
    assert more["weights"] == base["weights"] and more["cache"] == base["cache"]


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-q5k"])
def test_session_estimate_without_expanded_planes(name, monkeypatch):
    """BRISK_HIP_PREFILL_MX=0 (every format on the packed-plane GEMMs) drops exactly the Q6_K and
    Q5_K layer matrices' expanded planes from the estimate."""
    from brisk_hip.session import estimate
    f, cfg, table = model.load(synth.model_path(name))
    monkeypatch.delenv("BRISK_HIP_PREFILL_Q4X", raising=False)
    monkeypatch.delenv("BRISK_HIP_PREFILL_MX", raising=False)
    base = estimate((f, cfg, table), 256)
    monkeypatch.setenv("BRISK_HIP_PREFILL_MX", "0")
    less = estimate((f, cfg, table), 256)
    want = sum(_mx_bytes(t.type, t.rows, t.cols) for t in table
               if t.type in (G.T_Q6_K, G.T_Q5_K) and t.name.startswith("blk.") and t.rows > 1)
    assert want > 0
    assert base["scratch"] - less["scratch"] == want
