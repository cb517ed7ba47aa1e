"""CPU tests of the oracle (oracle/oracle.c) — no GPU.

The oracle is the checker the GPU parity tests compare against, so it is
pinned here three ways:
  * against the reference's own tests' known answers (tests/kernels_test.cpp:26-47)
    and its tolerance contract for every weight format (:96-184);
  * against library routines and closed forms: numpy's IEEE half conversion,
    brute-force integer block dots from dequantised weights, rms_norm of a
    constant vector, softmax invariants;
  * bit for bit against the reference itself where oracle/_ref is built (the
    reference engine compiled from its sources), function by function and on
    whole tiny models.
"""
import json
import os

import numpy as np
import pytest

import pyoracle
from pyoracle import ptr
from brisk_hip import gguf as G, model, synth

HERE = os.path.dirname(os.path.abspath(__file__))
needs_ref = pytest.mark.skipif(not pyoracle.ref_available(), reason="oracle/_ref is not built (no /root/reference)")

TYPES = (G.T_Q4_0, G.T_Q8_0, G.T_Q4_K, G.T_Q6_K, G.T_TQ2_0, G.T_Q4_1, G.T_Q5_0, G.T_Q5_K)
QK_BYTES = {G.T_Q4_0: 18, G.T_Q8_0: 34, G.T_Q4_K: 144, G.T_Q6_K: 210, G.T_TQ2_0: 66, G.T_Q4_1: 20, G.T_Q5_0: 22,
            G.T_Q5_K: 176}
SMALL = (G.T_Q4_0, G.T_Q8_0, G.T_Q4_1, G.T_Q5_0)  # 32-value blocks, Q8_0 activations


@pytest.fixture(scope="module")
def L():
    return pyoracle.oracle_lib()


def rng_normal(seed, n):
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


def q8_bytes(t):
    return 34 if t in SMALL else 292


def quantize(L, t, x, bits=8):
    blocks = len(x) // (32 if t in SMALL else 256)
    out = np.zeros(blocks * q8_bytes(t), np.uint8)
    if t in SMALL:
        L.or_quantize_q8_0(ptr(x), ptr(out), len(x))
    else:
        L.or_quantize_q8_k(ptr(x), ptr(out), len(x), bits)
    return out


# --------------------------------------------------------------------------- half conversion

def test_half_to_float_matches_ieee_half_exhaustively(L):
    """Every 16-bit pattern widens exactly as IEEE binary16 (numpy's float16)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.or_half_to_float(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_round_trips_and_rounds_to_even(L):
    """tests/kernels_test.cpp:26-38: round trip of every non-NaN half, the RNE tie cases, overflow, underflow."""
    for h in range(65536):
        f = L.or_half_to_float(h)
        if f != f:
            continue
        assert L.or_float_to_half(f) == h, hex(h)
    assert L.or_float_to_half(1.0 + 1.0 / 2048) == 0x3C00
    assert L.or_float_to_half(1.0 + 3.0 / 2048) == 0x3C02
    assert L.or_float_to_half(65520.0) == 0x7C00
    assert L.or_float_to_half(1e-8) == 0


def test_float_to_half_matches_numpy_on_random_floats(L):
    bits = np.random.default_rng(3).integers(0, 2**32, 60000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    got = np.array([L.or_float_to_half(float(v)) for v in f], np.uint16)
    assert np.array_equal(got, want)


# --------------------------------------------------------------------------- activation quantisation

def test_quantize_q8_0_known_answer(L):
    """tests/kernels_test.cpp:40-47."""
    x = ((np.arange(32) - 16) * 0.5).astype(np.float32)
    q = quantize(L, G.T_Q8_0, x)
    d = int(q[0]) | (int(q[1]) << 8)
    qs = q[2:34].view(np.int8)
    assert d == L.or_float_to_half(np.float32(8.0) / np.float32(127))
    assert qs[0] == -127 and qs[16] == 0 and qs[31] == 119


def test_quantize_q8_0_reconstructs_within_half_a_step(L):
    x = rng_normal(5, 4096) * 3
    q = quantize(L, G.T_Q8_0, x).reshape(-1, 34)
    d = q[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    qs = q[:, 2:].view(np.int8).astype(np.float32)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    # the stored scale is amax/127 rounded to half; q = rint(x / (amax/127)) in [-127, 127]
    assert np.all(np.abs(qs) <= 127)
    assert np.all(np.abs(qs).max(axis=1) == 127)
    err = np.abs(qs * (amax / 127)[:, None] - x.reshape(-1, 32))
    assert np.all(err <= (amax / 127)[:, None] * 0.5 + 1e-6)
    np.testing.assert_allclose(d, amax / 127, rtol=1e-3)


@pytest.mark.parametrize("bits", [8, 7])
def test_quantize_q8_k_invariants(L, bits):
    """Q8_K: the largest-magnitude value maps to -(2^(bits-1) - 1) sign-flipped, bsums are the sums of 16."""
    x = rng_normal(11 + bits, 2048)
    q = quantize(L, G.T_Q4_K, x, bits).reshape(-1, 292)
    d = q[:, 0:4].copy().view(np.float32).reshape(-1)
    qs = q[:, 4:260].view(np.int8).astype(np.int32)
    bsums = q[:, 260:292].copy().view(np.int16).astype(np.int32)
    assert np.array_equal(bsums, qs.reshape(-1, 16, 16).sum(axis=2))
    xb = x.reshape(-1, 256)
    i = np.argmax(np.abs(xb), axis=1)
    extreme = 63 if bits == 7 else 127
    assert np.all(qs[np.arange(len(i)), i] == -extreme)
    np.testing.assert_allclose(d[:, None] * qs, xb, atol=float(np.max(np.abs(d))) * 0.51 + 1e-6)


@needs_ref
@pytest.mark.parametrize("bits", [8, 7])
def test_quantize_matches_reference(L, bits):
    R = pyoracle.ref_lib()
    for seed in range(4):
        x = rng_normal(100 + seed, 6912 * 2 // 256 * 256) * (seed + 0.5)
        x[7] = 0.0
        a = np.zeros(len(x) // 32 * 34, np.uint8)
        b = np.zeros_like(a)
        L.or_quantize_q8_0(ptr(x), ptr(a), len(x))
        R.ref_quantize_q8_0(ptr(x), ptr(b), len(x))
        assert np.array_equal(a, b)
        a = np.zeros(len(x) // 256 * 292, np.uint8)
        b = np.zeros_like(a)
        L.or_quantize_q8_k(ptr(x), ptr(a), len(x), bits)
        R.ref_quantize_q8_k(ptr(x), ptr(b), len(x), bits)
        assert np.array_equal(a, b)
    z = np.zeros(512, np.float32)  # all-zero blocks: d = 0, q = 0
    a = np.ones(2 * 292, np.uint8)
    L.or_quantize_q8_k(ptr(z), ptr(a), 512, bits)
    assert not a.any()
    # an all-NaN block (the scan never picks a NaN: zeros) and equal magnitudes, the first negative
    x = rng_normal(9, 512) * 0.01
    x[:256] = np.nan
    x[256 + 7], x[256 + 100] = -5.0, 5.0
    a = np.zeros(2 * 292, np.uint8)
    b = np.zeros_like(a)
    L.or_quantize_q8_k(ptr(x), ptr(a), 512, bits)
    R.ref_quantize_q8_k(ptr(x), ptr(b), 512, bits)
    assert np.array_equal(a, b) and not a[:292].any()


# --------------------------------------------------------------------------- weights: dequant, dots

def weights(t, rows, cols, seed):
    be = 32 if t in SMALL else 256
    return synth.BLOCK_MAKERS[t](seed, rows * cols // be).reshape(-1)


def dequant(L, t, w, n):
    out = np.zeros(n, np.float32)
    L.or_dequantize(t, ptr(w), ptr(out), n)
    return out


def test_dequantize_q4_0_and_q8_0_closed_form(L):
    """Q4_0: (nibble - 8) * d with low nibbles first; Q8_0: int8 * d (src/quant.cpp:196-239)."""
    w = weights(G.T_Q4_0, 4, 64, 1).reshape(-1, 18)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32)
    qs = w[:, 2:]
    vals = np.concatenate([(qs & 0xF).astype(np.int32), (qs >> 4).astype(np.int32)], axis=1) - 8
    assert np.array_equal(dequant(L, G.T_Q4_0, w.reshape(-1), 256), (vals * d).astype(np.float32).reshape(-1))
    w = weights(G.T_Q8_0, 4, 64, 2).reshape(-1, 34)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32)
    vals = w[:, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal(dequant(L, G.T_Q8_0, w.reshape(-1), 256), (vals * d).reshape(-1))


def test_dequantize_q4_1_and_q5_0_closed_form(L):
    """Q4_1: q d + m; Q5_0: (nibble | fifth bit << 4) - 16, times d, the fifth bit of element e
    at bit e of qh (src/quant.cpp:207-232)."""
    w = weights(G.T_Q4_1, 4, 64, 11).reshape(-1, 20)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32)
    m = w[:, 2:4].copy().view(np.float16).astype(np.float32)
    qs = w[:, 4:]
    q = np.concatenate([(qs & 0xF), (qs >> 4)], axis=1).astype(np.float32)
    assert np.array_equal(dequant(L, G.T_Q4_1, w.reshape(-1), 256), (q * d + m).astype(np.float32).reshape(-1))
    w = weights(G.T_Q5_0, 4, 64, 12).reshape(-1, 22)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32)
    qh = w[:, 2:6].copy().view(np.uint32).astype(np.int64)
    qs = w[:, 6:].astype(np.int64)
    e = np.arange(32)
    nib = np.concatenate([qs & 0xF, qs >> 4], axis=1)
    q = nib | (((qh >> e) & 1) << 4)
    assert np.array_equal(dequant(L, G.T_Q5_0, w.reshape(-1), 256), ((q - 16).astype(np.float32) * d).reshape(-1))


def test_dequantize_tq2_0_is_ternary(L):
    w = weights(G.T_TQ2_0, 2, 512, 3)
    v = dequant(L, G.T_TQ2_0, w, 1024)
    d = np.float32(w[64:66].copy().view(np.float16)[0])
    assert set(np.unique(v / d).tolist()) <= {-1.0, 0.0, 1.0}


@needs_ref
@pytest.mark.parametrize("t", TYPES)
def test_dequantize_matches_reference(L, t):
    R = pyoracle.ref_lib()
    w = weights(t, 8, 1024, 7)
    a = dequant(L, t, w, 8 * 1024)
    b = np.zeros_like(a)
    R.ref_dequantize(t, ptr(w), ptr(b), len(b))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def int_block_dots(L, t, w, xq, cols):
    """Brute force: per block, the exact integer sum of (weight integer) x (activation integer),
    both recovered from dequantisation (weights) or the raw bytes (activations)."""
    if t in (G.T_Q4_0, G.T_Q8_0, G.T_Q5_0):
        nb = cols // 32
        wb = w.reshape(nb, -1)
        wd = wb[:, 0:2].copy().view(np.float16).astype(np.float32)
        deq = dequant(L, t, w, cols).reshape(nb, 32)
        wi = np.rint(deq / wd).astype(np.int64)
        xb = xq.reshape(nb, 34)
        xi = xb[:, 2:].view(np.int8).astype(np.int64)
        return (wi * xi).sum(axis=1)
    return None


@pytest.mark.parametrize("t", [G.T_Q4_0, G.T_Q8_0, G.T_Q5_0])
def test_block_dot_equals_brute_force(L, t):
    """or_dot = sequential fp32 sum of float(int block dot) * d_w * d_x (src/quant.cpp:445-482)."""
    cols = 1024
    for seed in range(3):
        w = weights(t, 1, cols, 20 + seed)
        x = rng_normal(30 + seed, cols)
        xq = quantize(L, t, x)
        acc = int_block_dots(L, t, w, xq, cols)
        wd = w.reshape(cols // 32, -1)[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
        xd = xq.reshape(cols // 32, 34)[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
        s = np.float32(0)
        for b in range(cols // 32):
            s = np.float32(s + np.float32(np.float32(acc[b]) * wd[b]) * xd[b])
        assert L.or_dot(t, 0, ptr(w), ptr(xq), cols // 32) == s


@pytest.mark.parametrize("t", TYPES)
def test_matvec_within_reference_tolerance(L, t):
    """tests/kernels_test.cpp:96-184: every row within activation rounding of the double
    dot of its dequantised weights with the unquantised x."""
    rows, cols = 37, 1024
    w = weights(t, rows, cols, 41)
    x = rng_normal(42, cols)
    bits = 7 if (t == G.T_TQ2_0 and rows % 16 == 0) else 8
    xq = quantize(L, t, x, bits)
    out = np.zeros(rows, np.float32)
    L.or_matvec(t, ptr(w), rows, cols, ptr(xq), ptr(out))
    deq = dequant(L, t, w, rows * cols).reshape(rows, cols).astype(np.float64)
    ref = deq @ x.astype(np.float64)
    step = 126.0 if bits == 7 else 254.0
    tol = 0.02 + 4.0 * np.linalg.norm(deq, axis=1) * np.abs(x).max() / step
    assert np.all(np.abs(out - ref) <= tol)


@needs_ref
@pytest.mark.parametrize("t,rows", [(G.T_Q4_0, 37), (G.T_Q8_0, 37), (G.T_Q4_K, 37), (G.T_Q6_K, 37),
                                    (G.T_TQ2_0, 37), (G.T_TQ2_0, 48), (G.T_Q4_1, 37), (G.T_Q5_0, 37),
                                    (G.T_Q5_K, 37)])
def test_matvec_matches_reference_bitwise(L, t, rows):
    R = pyoracle.ref_lib()
    cols = 2048
    w = weights(t, rows, cols, 50 + rows)
    lut16 = t == G.T_TQ2_0 and rows % 16 == 0
    bits = 7 if lut16 else 8
    for seed in range(3):
        x = rng_normal(60 + seed, cols)
        xq = quantize(L, t, x, bits)
        a = np.zeros(rows, np.float32)
        b = np.zeros(rows, np.float32)
        L.or_matvec(t, ptr(w), rows, cols, ptr(xq), ptr(a))
        if lut16:
            packed = np.zeros(rows // 16 * (cols // 256) * 1056, np.uint8)
            R.ref_repack_tq2_0x16(ptr(w), rows, cols // 256, ptr(packed))
            assert R.ref_matvec(1016, ptr(packed), rows, cols, ptr(xq), ptr(b)) == 0
        else:
            assert R.ref_matvec(t, ptr(w), rows, cols, ptr(xq), ptr(b)) == 0
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@needs_ref
def test_tq2_0x16_repack_matches_reference(L):
    R = pyoracle.ref_lib()
    rows, cols = 48, 1024
    w = weights(G.T_TQ2_0, rows, cols, 77)
    a = np.zeros(rows // 16 * (cols // 256) * 1056, np.uint8)
    b = np.zeros_like(a)
    L.or_repack_tq2_0x16(ptr(w), rows, cols // 256, ptr(a))
    R.ref_repack_tq2_0x16(ptr(w), rows, cols // 256, ptr(b))
    assert np.array_equal(a, b)


def test_activation_bits(L):
    """7-bit activations exactly for TQ2_0 matrices with a multiple of 16 rows (src/model.cpp:496-503)."""
    assert L.or_activation_bits(G.T_TQ2_0, 2560) == 7
    assert L.or_activation_bits(G.T_TQ2_0, 37) == 8
    assert L.or_activation_bits(G.T_Q4_K, 2048) == 8


# --------------------------------------------------------------------------- float kernels

def test_dot_f32_lane_order(L):
    """dot_f32: 16 lane partials over i = j mod 16, then the tail, then lanes 0..15 (src/kernels_f32.cpp:229-246)."""
    for n in (16, 128, 77):
        a, b = rng_normal(n, n), rng_normal(n + 1, n)
        lanes = np.zeros(16, np.float32)
        full = n // 16 * 16
        for i in range(full):
            lanes[i % 16] = np.float32(lanes[i % 16] + np.float32(a[i] * b[i]))
        s = np.float32(0)
        for i in range(full, n):
            s = np.float32(s + np.float32(a[i] * b[i]))
        for j in range(16):
            s = np.float32(s + lanes[j])
        assert L.or_dot_f32(ptr(a), ptr(b), n) == s
        assert abs(float(s) - float(a.astype(np.float64) @ b.astype(np.float64))) < 1e-4 * n


def test_softmax_invariants(L):
    x = rng_normal(9, 300) * 4
    y = x.copy()
    L.or_softmax(ptr(y), len(y))
    assert abs(float(y.astype(np.float64).sum()) - 1.0) < 1e-5
    assert int(np.argmax(y)) == int(np.argmax(x))
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(y, e / e.sum(), rtol=2e-6, atol=1e-9)
    c = np.full(8, 3.0, np.float32)  # uniform input: exactly 1/8 each
    L.or_softmax(ptr(c), 8)
    assert np.all(c == np.float32(0.125))


@needs_ref
def test_float_kernels_match_reference(L):
    R = pyoracle.ref_lib()
    for n in (64, 128, 333):
        a, b = rng_normal(n, n), rng_normal(n + 7, n)
        assert L.or_dot_f32(ptr(a), ptr(b), n) == R.ref_dot_f32(ptr(a), ptr(b), n)
        x = rng_normal(n + 9, n) * 5
        y1, y2 = x.copy(), x.copy()
        L.or_softmax(ptr(y1), n)
        R.ref_softmax(ptr(y2), n)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_rms_norm_closed_form(L):
    """rms_norm of a constant vector c is c / sqrt(c^2 + eps) * w (src/model.cpp:87-97)."""
    n, eps = 1024, 1e-6
    x = np.full(n, 0.75, np.float32)
    w = rng_normal(4, n)
    out = np.zeros(n, np.float32)
    L.or_rms_norm(ptr(x), ptr(w), np.float32(eps), ptr(out), n)
    scale = np.float32(1.0) / np.sqrt(np.float32(np.float32(0.5625) + np.float32(eps)))
    assert np.array_equal(out, (x * scale * w).astype(np.float32))
    x = rng_normal(5, n)
    L.or_rms_norm(ptr(x), ptr(w), np.float32(eps), ptr(out), n)
    want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps) * w
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=1e-7)


def test_expf_restatement_matches_libm():
    """The HIP loop's expf restatement (glibc's table + polynomial) against the host libm, on a strided sweep
    of every float bit pattern."""
    import ctypes as C
    L = pyoracle.oracle_lib()
    checked = C.c_uint64()
    bad = L.or_expf_check(997, C.byref(checked))
    assert checked.value > 4_000_000
    assert bad == 0


def test_tanhf_restatement_matches_libm():
    """The Gemma epilogues' tanhf restatement (fdlibm's tanhf over expm1f, as glibc 2.35 builds it) against the
    host libm, on a strided sweep of every float bit pattern (every pattern when run with stride 1)."""
    import ctypes as C
    L = pyoracle.oracle_lib()
    checked = C.c_uint64()
    bad = L.or_tanhf_check(997, C.byref(checked))
    assert checked.value > 4_000_000
    assert bad == 0


def test_log1pf_restatement_matches_libm():
    """The Qwen3.5 recurrence's log1pf restatement (fdlibm's s_log1pf.c, as glibc 2.35 builds it) against the
    host libm, on a strided sweep of every float bit pattern (every pattern agrees when run with stride 1)."""
    import ctypes as C
    L = pyoracle.oracle_lib()
    checked = C.c_uint64()
    bad = L.or_log1pf_check(97, C.byref(checked))
    assert checked.value > 40_000_000
    assert bad == 0


def test_log1pf_closed_forms():
    """log1p at its special points and where it reduces to a textbook value: log1p(0) = 0, log1p(e - 1) = 1,
    log1p(-1) = -inf, log1p(x) = x for tiny x, log1p(2^k - 1) = k ln 2."""
    import ctypes as C
    L = pyoracle.oracle_lib()
    x = np.array([0.0, np.e - 1, -1.0, 1e-30, 1.0, 3.0, 7.0, 1023.0], np.float32)
    y = np.empty_like(x)
    L.or_log1pf_batch(pyoracle.ptr(x), pyoracle.ptr(y), len(x))
    assert y[0] == 0.0 and abs(y[1] - 1.0) <= 1.2e-7 and y[2] == -np.inf and y[3] == np.float32(1e-30)
    for i, k in ((4, 1), (5, 2), (6, 3), (7, 10)):
        assert abs(float(y[i]) - k * np.log(2.0)) <= 1e-6 * k


# --------------------------------------------------------------------------- whole models

def tiny(name):
    path = synth.model_path(name)
    f, cfg, table = model.load(path)
    return path, f, cfg, table


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama", "tiny-q8", "tiny-bitnet", "tiny-q5k", "tiny-q5", "tiny-qwen2", "tiny-smollm3", "tiny-gemma3", "tiny-phi3", "tiny-llama32", "tiny-lfm2", "tiny-qwen35", "tiny-qwen35w", "tiny-qwen35h", "tiny-gemma4"])
def test_oracle_greedy_matches_reference_fixture(name):
    """tests/golden/<name>_greedy.json were written by the reference engine itself."""
    with open(os.path.join(HERE, "golden", f"{name}_greedy.json")) as fh:
        g = json.load(fh)
    path, f, cfg, table = tiny(name)
    o = pyoracle.Oracle(cfg, table, max_context=len(g["prompt"]) + len(g["ids"]) + 4)
    logits = o.eval(np.array(g["prompt"], np.int32))
    pl = g["prompt_logits"]
    assert np.array_equal(logits[::61], np.array(pl["every61"], np.float32))
    assert np.array_equal(logits[pl["top_idx"]], np.array(pl["top_val"], np.float32))
    o.rollback(0)
    ids, _ = o.generate(np.array(g["prompt"], np.int32), len(g["ids"]))
    assert ids.tolist() == g["ids"]
    o.close()


def test_oracle_first_tokens_of_qwen3_0_6b_fixture():
    """configs[1] at full size: the first greedy ids of the reference's 256-step run."""
    with open(os.path.join(HERE, "golden", "qwen3-0.6b_greedy.json")) as fh:
        g = json.load(fh)
    path, f, cfg, table = tiny("qwen3-0.6b")
    o = pyoracle.Oracle(cfg, table, max_context=64)
    ids, _ = o.generate(np.array(g["prompt"], np.int32), 3)
    assert ids.tolist() == g["ids"][:3]
    o.close()


@needs_ref
@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama", "tiny-bitnet", "tiny-q5k", "tiny-q5", "tiny-qwen2", "tiny-smollm3", "tiny-gemma3", "tiny-phi3", "tiny-llama32", "tiny-lfm2", "tiny-qwen35", "tiny-qwen35w", "tiny-qwen35h", "tiny-gemma4"])
def test_oracle_session_matches_reference_bitwise(name):
    """eval, eval_all and rollback of the restatement against the reference's Session."""
    path, f, cfg, table = tiny(name)
    prompt = synth.prompt_ids(20, cfg.vocab, seed=3)
    o = pyoracle.Oracle(cfg, table, max_context=64)
    r = pyoracle.Reference(path, threads=2, max_context=64)
    a, b = o.eval(prompt), r.eval(prompt)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    o.rollback(7)
    r.rollback(7)
    a = o.eval(prompt[7:12], all_logits=True)
    b = r.eval_all(prompt[7:12])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # Qwen3.5's recurrent states cannot step back to 7: the rollback restarted them at 0
    assert o.position == r.position == (5 if cfg.arch == model.ARCH_QWEN35 else 12)
    o.close()
    r.close()


@needs_ref
@pytest.mark.parametrize("name", ["tiny-qwen35", "tiny-qwen35w", "tiny-qwen35h"])
def test_oracle_recurrent_snapshot_matches_reference_bitwise(name):
    """Qwen3.5's rollback (src/model.cpp:735-752): one step back restores the snapshot taken before the last
    token, whether that token came alone or at the end of a longer call; a second step back, or any other
    earlier position, restarts at 0; rolling back to the current position changes nothing."""
    path, f, cfg, table = tiny(name)
    prompt = synth.prompt_ids(20, cfg.vocab, seed=5)
    o = pyoracle.Oracle(cfg, table, max_context=64)
    r = pyoracle.Reference(path, threads=2, max_context=64)
    same = lambda a, b: np.array_equal(a.view(np.uint32), b.view(np.uint32))  # noqa: E731
    first = o.eval(prompt[:10])
    assert same(first, r.eval(prompt[:10]))
    for h in (o, r):
        h.rollback(10)  # the current position: nothing happens
        h.rollback(9)   # the snapshot before the call's last token
    assert o.position == r.position == 9
    a, b = o.eval(prompt[9:10]), r.eval(prompt[9:10])
    assert same(a, b) and same(a, first)  # the token again from the restored state
    a, b = o.eval(prompt[10:11]), r.eval(prompt[10:11])
    assert same(a, b)
    for h in (o, r):
        h.rollback(10)
    again = o.eval(prompt[10:11])
    assert same(again, r.eval(prompt[10:11])) and same(again, a)
    for h in (o, r):
        h.rollback(10)
        h.rollback(9)   # the snapshot was used: a restart
    assert o.position == r.position == 0
    a, b = o.eval(prompt[:4], all_logits=True), r.eval_all(prompt[:4])
    assert same(a, b)
    for h in (o, r):
        h.rollback(1)   # not the snapshot's position (3): a restart
    assert o.position == r.position == 0
    o.close()
    r.close()


@needs_ref
def test_oracle_longrope_matches_reference_bitwise():
    """Phi-3 with a context past rope.scaling.original_context_length takes the long factors
    (src/model.cpp:691-694): the restatement against the reference's Session at 600 positions."""
    path, f, cfg, table = tiny("tiny-phi3")
    prompt = synth.prompt_ids(20, cfg.vocab, seed=3)
    o = pyoracle.Oracle(cfg, table, max_context=600)
    r = pyoracle.Reference(path, threads=2, max_context=600)
    a, b = o.eval(prompt), r.eval(prompt)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    short = pyoracle.Oracle(cfg, table, max_context=64)
    assert not np.array_equal(short.eval(prompt), a)  # the factors differ, so the logits do
    o.close()
    r.close()
    short.close()


@needs_ref
@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama", "tiny-bitnet", "tiny-q5k", "tiny-q5", "tiny-qwen2", "tiny-smollm3", "tiny-gemma3", "tiny-phi3", "tiny-llama32", "tiny-lfm2", "tiny-qwen35", "tiny-qwen35w", "tiny-qwen35h", "tiny-gemma4"])
def test_model_config_matches_reference(name):
    """brisk_hip.model.parse_config against the reference's own ModelConfig parse (src/model.cpp:140-260)
    of the same file, field by field. The Python config keeps 0 for a field its family does not use;
    the reference holds its default there (src/model.h:34-125), so those map through the defaults."""
    path, f, cfg, table = tiny(name)
    r = pyoracle.Reference(path, threads=1, max_context=16)
    c = r.config()
    r.close()
    assert c.arch == pyoracle.REF_ARCH[cfg.arch_name]
    assert (c.vocab, c.embd, c.layers, c.heads, c.kv_heads, c.head_dim, c.ff, c.context) == \
        (cfg.vocab, cfg.embd, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.ff, cfg.context)
    f32 = lambda x: np.float32(x).view(np.uint32)  # noqa: E731
    assert f32(c.rope_base) == f32(cfg.rope_base) and f32(c.eps) == f32(cfg.eps)
    assert bool(c.rope_neox) == cfg.rope_neox
    assert c.rope_dim == (cfg.rope_dim or cfg.head_dim)
    assert c.rope_original_context == cfg.rope_original_context
    assert f32(c.rope_attn_factor) == f32(cfg.rope_attn_factor or 1.0)
    assert c.sliding_window == cfg.sliding_window
    gemma = cfg.arch in (model.ARCH_GEMMA3, model.ARCH_GEMMA4)
    assert f32(c.rope_base_local) == f32(cfg.rope_base_local if gemma else 10000.0)
    assert f32(c.rope_scale) == f32(cfg.rope_scale if gemma else 1.0)
    assert f32(c.final_softcap) == f32(cfg.final_softcap)
    # Gemma's sqrt(embedding_dim) input scale and GELU activation follow from the family in the session
    assert f32(c.embedding_scale) == f32(np.sqrt(np.float32(cfg.embd)) if gemma else 1.0)
    assert bool(c.gelu) == gemma
    assert c.conv_taps == cfg.conv_taps
    # layer_is_conv (src/model.h:95) holds for every layer without key/value heads, Qwen3.5's recurrent
    # ones included; eval_batch asks layer_is_recurrent first (src/model.cpp:932-934)
    assert c.conv_layers == sum(1 << l for l in cfg.conv_layers + cfg.recurrent_layers)
    assert c.recurrent_layers == sum(1 << l for l in cfg.recurrent_layers)
    assert (c.ssm_state, c.ssm_k_heads, c.ssm_v_heads, c.ssm_inner, c.ssm_conv) == \
        (cfg.ssm_state, cfg.ssm_k_heads, cfg.ssm_v_heads, cfg.ssm_inner, cfg.ssm_conv)
    assert bool(c.attention_gate) == (cfg.arch == model.ARCH_QWEN35)
    # Gemma 4's per-layer shapes (src/model.h:76-118)
    assert (c.head_dim_local, c.kv_from_start, c.ple_dim, bool(c.value_norm)) == \
        (cfg.head_dim_local, cfg.kv_from_start, cfg.ple_dim, bool(cfg.value_norm))
    assert f32(c.attention_scale) == f32(cfg.attention_scale)
    for l in range(cfg.layers):
        assert bool(c.sliding_layers >> l & 1) == (cfg.layer_slides(l) if cfg.arch in (model.ARCH_GEMMA3, model.ARCH_GEMMA4)
                                                   else False), l
        assert (c.head_dim_of[l], c.ff_of[l], c.kv_layer_of[l]) == (cfg.head_dim_of(l), cfg.ff_of(l), cfg.kv_layer_of(l)), l
        if l not in cfg.conv_layers + cfg.recurrent_layers:
            assert c.kv_heads_of[l] == cfg.kv_heads_of(l), l
    assert c.no_rope_step == (4 if cfg.arch == model.ARCH_SMOLLM3 else 0)
    assert [l for l in range(cfg.layers) if not cfg.layer_has_rope(l)] == \
        ([l for l in range(cfg.layers) if (l + 1) % c.no_rope_step == 0] if c.no_rope_step else [])
    names = {t.name for t in table}
    # Phi-3 starts from its short LongRoPE factors (src/model.cpp:186)
    assert (c.n_rope_factors > 0) == ("rope_freqs.weight" in names or "rope_factors_short.weight" in names)
    assert (c.n_factors_short > 0) == (c.n_factors_long > 0) == ("rope_factors_short.weight" in names)


def test_oracle_rejects_bad_input():
    path, f, cfg, table = tiny("tiny-qwen3")
    o = pyoracle.Oracle(cfg, table, max_context=8)
    with pytest.raises(RuntimeError, match="no tokens"):
        o.eval(np.array([], np.int32))
    with pytest.raises(RuntimeError, match="out of range"):
        o.eval(np.array([cfg.vocab], np.int32))
    with pytest.raises(RuntimeError, match="context length"):
        o.eval(np.arange(9, dtype=np.int32))
    o.eval(np.arange(3, dtype=np.int32))
    with pytest.raises(RuntimeError, match="roll forward"):
        o.rollback(5)
    o.close()
