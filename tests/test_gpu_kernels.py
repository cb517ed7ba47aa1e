"""GPU parity of the kernel-level ABI against the oracle (bit-exact).

The oracle's functions are themselves bit-identical to the reference's
(tests/test_oracle.py), so equality here is equality with the reference's
quantize_q8_0 / quantize_q8_k / generic matvec and matmul (src/quant.cpp,
src/kernels.cpp).  Shapes follow the reference's kernels_test (37 rows x 1024
columns, 7 tokens, src/../tests/kernels_test.cpp:186-225) plus config 1's
2048 x 2048 Q4_0 matrix and the widths of the benchmark models.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import lib as L  # noqa: E402
from brisk_hip import synth  # noqa: E402
import pyoracle  # noqa: E402

Q4_0, Q4_1, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ2_0 = 2, 3, 6, 8, 12, 13, 14, 35
BLOCK = {Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210), TQ2_0: (256, 66)}
Q8K = (Q4_K, Q5_K, Q6_K, TQ2_0)


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()


def p(t):
    return C.c_void_p(t.data_ptr())


def host(t, dtype):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(dtype)


@pytest.fixture(scope="module")
def lib():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return L.load()


@pytest.fixture(scope="module")
def orc():
    return pyoracle.oracle_lib()


def weights(type_, rows, cols, seed):
    be, bb = BLOCK[type_]
    return synth.BLOCK_MAKERS[type_](seed, rows * cols // be).reshape(-1)


def activations(n, seed, scale=1.0):
    return (synth.random_normalish(seed, n) * scale).astype(np.float32)


def quant_ref(orc, x, q8k, bits=8):
    if q8k:
        out = np.zeros(len(x) // 256 * 292, np.uint8)
        orc.or_quantize_q8_k(pyoracle.ptr(x), pyoracle.ptr(out), len(x), bits)
    else:
        out = np.zeros(len(x) // 32 * 34, np.uint8)
        orc.or_quantize_q8_0(pyoracle.ptr(x), pyoracle.ptr(out), len(x))
    return out


@pytest.mark.parametrize("n", [32, 1024, 8192, 8192 * 3 + 4096])
def test_quantize_q8_0_bitexact(lib, orc, n):
    x = activations(n, n)
    if n >= 96:
        x[:32] = 0.0                                        # an all-zero block: d = 0
        x[64:96] = np.arange(32, dtype=np.float32) - 15.5   # values that scale to exact .5 ties
    want = quant_ref(orc, x, False)
    xd = dev(x)
    out = torch.zeros(len(want), dtype=torch.uint8, device="cuda")
    L.check(lib.brisk_hip_quantize_q8_0(p(xd), p(out), n, None))
    np.testing.assert_array_equal(host(out, np.uint8), want)


@pytest.mark.parametrize("bits", [8, 7])
@pytest.mark.parametrize("n", [256, 2560, 8192, 8192 + 2048])
def test_quantize_q8_k_bitexact(lib, orc, n, bits):
    x = activations(n, n + bits)
    if n >= 512:
        x[:256] = 0.0
        x[256 + 10] = -7.0
        x[256 + 20] = 7.0   # equal magnitude later: the first one (negative) sets the scale
    want = quant_ref(orc, x, True, bits)
    xd = dev(x)
    out = torch.zeros(len(want), dtype=torch.uint8, device="cuda")
    L.check(lib.brisk_hip_quantize_q8_k(p(xd), p(out), n, bits, None))
    np.testing.assert_array_equal(host(out, np.uint8), want)


@pytest.mark.parametrize("bits", [8, 7])
def test_quantize_q8_k_special_blocks(lib, orc, bits):
    """Blocks whose scale value the wave search must pick as the reference's scan does: all NaN
    (the scan never picks a NaN, so the block is zeros), equal magnitudes in different lanes (the
    first, negative, sets the scale), zeros with -0.0, and an ordinary block."""
    x = activations(1024, 40 + bits)
    x[:256] = np.nan
    x[256:512] *= 0.01
    x[256 + 7] = -5.0
    x[256 + 100] = 5.0
    x[256 + 201] = -5.0
    x[512:768] = 0.0
    x[512 + 3::17] = -0.0
    want = quant_ref(orc, x, True, bits)
    xd = dev(x)
    out = torch.zeros(len(want), dtype=torch.uint8, device="cuda")
    L.check(lib.brisk_hip_quantize_q8_k(p(xd), p(out), 1024, bits, None))
    np.testing.assert_array_equal(host(out, np.uint8), want)


def packed(lib, type_, w, rows, cols):
    nbytes = lib.brisk_hip_packed_bytes(type_, rows, cols)
    assert nbytes > 0
    src = dev(w)
    dst = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    L.check(lib.brisk_hip_pack(type_, p(src), rows, cols, p(dst), None))
    return dst


CASES = [
    (Q4_0, 37, 1024), (Q4_0, 2048, 2048), (Q4_0, 1024, 3072), (Q4_0, 3072, 1024),
    (Q8_0, 37, 1024), (Q8_0, 2048, 6144), (Q8_0, 300, 2048),
    (Q4_K, 37, 1024), (Q4_K, 512, 2048), (Q4_K, 2048, 8192),
    (Q6_K, 37, 1024), (Q6_K, 512, 2048), (Q6_K, 2048, 8192), (Q6_K, 200, 256), (Q6_K, 130, 512), (Q6_K, 300, 1280),
    (TQ2_0, 48, 1024), (TQ2_0, 640, 2560), (TQ2_0, 37, 2560),
    (Q4_1, 37, 1024), (Q4_1, 2048, 2048), (Q5_0, 37, 1024), (Q5_0, 1024, 3072),
    (Q5_K, 37, 1024), (Q5_K, 512, 2048), (Q5_K, 2048, 8192),
    # rows wider than the GEMV's LDS row (4B-class feed-forward widths): the planar GEMM path, n = 1 too
    (Q4_0, 64, 14336), (Q8_0, 48, 9728), (Q4_K, 64, 9728), (Q6_K, 48, 14336), (TQ2_0, 48, 9728),
    (Q4_1, 37, 9728), (Q5_0, 37, 14336), (Q5_K, 37, 9728),
]


@pytest.mark.parametrize("n", [7, 67])  # batches run on int8 MFMA: 16-token groups, 64-token tiles
@pytest.mark.parametrize("type_,rows,cols", CASES)
def test_matvec_matmul_bitexact(lib, orc, type_, rows, cols, n):
    w = weights(type_, rows, cols, rows * 7919 + cols)
    q8k = type_ in Q8K
    bits = orc.or_activation_bits(type_, rows)
    xs = [activations(cols, 100 + t) for t in range(n)]
    xq = np.concatenate([quant_ref(orc, x, q8k, bits) for x in xs])
    rb = cols // BLOCK[type_][0] * (292 if q8k else 34)
    want = np.zeros((n, rows), np.float32)
    for t in range(n):
        orc.or_matvec(type_, pyoracle.ptr(w), rows, cols, pyoracle.ptr(xq[t * rb:(t + 1) * rb]), pyoracle.ptr(want[t]))
    flags = 1 if (type_ == TQ2_0 and rows % 16 == 0) else 0
    wd = packed(lib, type_, w, rows, cols)
    xd = dev(xq)
    out = torch.zeros(rows, dtype=torch.float32, device="cuda")
    L.check(lib.brisk_hip_matvec(type_, flags, p(wd), rows, cols, p(xd), p(out), None))
    np.testing.assert_array_equal(host(out, np.float32), want[0])
    out2 = torch.zeros(n * (rows + 3), dtype=torch.float32, device="cuda")
    L.check(lib.brisk_hip_matmul(type_, flags, p(wd), rows, cols, p(xd), n, p(out2), rows + 3, None))
    got = host(out2, np.float32).reshape(n, rows + 3)[:, :rows]
    np.testing.assert_array_equal(got, want)


def test_wide_rows_need_whole_chunks(lib):
    """Rows wider than 8192 go through 256-value chunks: a width that is not whole chunks is refused
    with an error (no launch); the fused-norm GEMV, which holds the row in LDS, refuses any wider row."""
    rows, cols = 37, 8192 + 32
    w = weights(Q4_0, rows, cols, 5)
    nbytes = lib.brisk_hip_packed_bytes(Q4_0, rows, cols)
    wd = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    assert lib.brisk_hip_pack(Q4_0, p(dev(w)), rows, cols, p(wd), None) != 0
    assert b"256-value blocks" in lib.brisk_hip_last_error()
    cols = 9728
    x = torch.zeros(cols, dtype=torch.float32, device="cuda")
    out = torch.zeros(rows, dtype=torch.float32, device="cuda")
    wd = torch.zeros(lib.brisk_hip_packed_bytes(Q4_0, rows, cols), dtype=torch.uint8, device="cuda")
    assert lib.brisk_hip_gemv(Q4_0, 0, p(wd), rows, cols, p(x), None, 1e-6, p(out), 0, None) != 0
    assert b"wider than 8192" in lib.brisk_hip_last_error()


@pytest.mark.parametrize("type_,rows,cols", [(Q4_0, 2048, 1024), (Q8_0, 4096, 1024), (Q4_K, 256, 2048),
                                              (Q6_K, 256, 8192), (TQ2_0, 640, 2560), (Q4_1, 2048, 1024),
                                              (Q5_0, 1024, 2048), (Q5_K, 256, 4096)])
def test_gemv_fused_norm_bitexact(lib, orc, type_, rows, cols):
    """In-kernel rms_norm + quantisation + matvec equals the oracle's rms_norm -> quantize -> matvec."""
    w = weights(type_, rows, cols, rows + cols)
    x = activations(cols, 5, 3.0)
    nw = synth.random_uniform(9, cols, 0.8, 1.2).astype(np.float32)
    eps = 1e-6
    normed = np.zeros(cols, np.float32)
    orc.or_rms_norm(pyoracle.ptr(x), pyoracle.ptr(nw), eps, pyoracle.ptr(normed), cols)
    bits = orc.or_activation_bits(type_, rows)
    xq = quant_ref(orc, normed, type_ in Q8K, bits)
    want = np.zeros(rows, np.float32)
    orc.or_matvec(type_, pyoracle.ptr(w), rows, cols, pyoracle.ptr(xq), pyoracle.ptr(want))
    flags = 1 if (type_ == TQ2_0 and rows % 16 == 0) else 0
    wd = packed(lib, type_, w, rows, cols)
    xd, nwd = dev(x), dev(nw)
    out = torch.zeros(rows, dtype=torch.float32, device="cuda")
    L.check(lib.brisk_hip_gemv(type_, flags, p(wd), rows, cols, p(xd), p(nwd), eps, p(out), 0, None))
    np.testing.assert_array_equal(host(out, np.float32), want)
    # accumulate: out += W x (the residual update)
    base = activations(rows, 77)
    acc = dev(base)
    L.check(lib.brisk_hip_gemv(type_, flags, p(wd), rows, cols, p(xd), p(nwd), eps, p(acc), 1, None))
    np.testing.assert_array_equal(host(acc, np.float32), base + want)


def test_errors_are_reported(lib):
    rc = lib.brisk_hip_matvec(Q4_0, 0, None, 16, 1000, None, None, None)
    assert rc == -1
    assert b"multiple of the block size" in lib.brisk_hip_last_error()


def test_expf_matches_host_libm(lib, orc):
    """The device expf used by softmax and SiLU equals glibc's expf (the reference's std::exp)."""
    bits = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    want = np.empty_like(x)
    orc.or_expf_batch(pyoracle.ptr(x), pyoracle.ptr(want), len(x))
    xd = dev(x)
    out = torch.zeros(len(x), dtype=torch.float32, device="cuda")
    L.check(lib.brisk_hip_expf(p(xd), p(out), len(x), None))
    got = host(out, np.float32)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert len(bad) == 0, f"{len(bad)} of {len(x)} differ, e.g. x={x[bad[:3]]} got={got[bad[:3]]} want={want[bad[:3]]}"


def test_tanhf_matches_host_libm(lib, orc):
    """The device tanhf used by the GELU gate and the logit softcap equals glibc's tanhf (the reference's std::tanh)."""
    bits = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    want = np.empty_like(x)
    orc.or_tanhf_batch(pyoracle.ptr(x), pyoracle.ptr(want), len(x))
    xd = dev(x)
    out = torch.zeros(len(x), dtype=torch.float32, device="cuda")
    L.check(lib.brisk_hip_tanhf(p(xd), p(out), len(x), None))
    got = host(out, np.float32)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert len(bad) == 0, f"{len(bad)} of {len(x)} differ, e.g. x={x[bad[:3]]} got={got[bad[:3]]} want={want[bad[:3]]}"


def test_log1pf_matches_host_libm(lib, orc):
    """The device log1pf of the Qwen3.5 recurrence's softplus equals glibc's log1pf (the reference's std::log1p):
    a strided sweep of every float pattern, and every float of [1, 2) and of [2^20, 2^21) (exp of the softplus
    inputs below its cut-over at 20 reaches 4.9e8)."""
    bits = np.concatenate([np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32),
                           np.arange(0x3F800000, 0x40000000, dtype=np.uint32),
                           np.arange(0x49800000, 0x4A000000, dtype=np.uint32)])
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    want = np.empty_like(x)
    orc.or_log1pf_batch(pyoracle.ptr(x), pyoracle.ptr(want), len(x))
    xd = dev(x)
    out = torch.zeros(len(x), dtype=torch.float32, device="cuda")
    L.check(lib.brisk_hip_log1pf(p(xd), p(out), len(x), None))
    got = host(out, np.float32)
    bad = np.flatnonzero((got.view(np.uint32) != want.view(np.uint32)) & ~(np.isnan(got) & np.isnan(want)))
    assert len(bad) == 0, f"{len(bad)} of {len(x)} differ, e.g. x={x[bad[:3]]} got={got[bad[:3]]} want={want[bad[:3]]}"


def test_short_divisions_are_exact(lib):
    """div127 (a / 127, a >= 0) and rcp_rn (1 / d) equal IEEE division on every finite input, and the
    hardware float-to-half conversion equals the reference's bit-level one on every float, and the
    one-instruction float x half product equals the product of the widened half on every float."""
    import ctypes
    bad = (ctypes.c_ulonglong * 4)()
    L.check(lib.brisk_hip_div_selftest(bad))
    assert list(bad) == [0, 0, 0, 0], f"div127: {bad[0]} mismatches, rcp_rn: {bad[1]}, f2h: {bad[2]}, mul_h: {bad[3]}"
