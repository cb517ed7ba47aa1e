"""The no-alloc matmul (brisk_hip_matmul_noalloc) against brisk_hip_matmul.

brisk_hip_matmul stages a batch's activation rows in a hipMalloc'd buffer; the
no-alloc entry point stages them in a static device buffer that every call on
the GPU reuses.  Two calls in a row, the second with a smaller batch, must each
give exactly brisk_hip_matmul's outputs (bit-exact), and a batch beyond the
buffer must be refused.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from brisk_hip import lib as L  # noqa: E402
from brisk_hip import synth  # noqa: E402
import pyoracle  # noqa: E402

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, TQ2_0 = 2, 8, 12, 13, 14, 35
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), TQ2_0: (256, 66)}
Q8K = (Q4_K, Q5_K, Q6_K, TQ2_0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()


def p(t):
    return C.c_void_p(t.data_ptr())


@pytest.fixture(scope="module")
def lib():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return L.load()


def quantised_rows(orc, type_, rows, cols, n, seed):
    q8k = type_ in Q8K
    bits = orc.or_activation_bits(type_, rows)
    out = []
    for t in range(n):
        x = synth.random_normalish(seed + t, cols).astype(np.float32)
        q = np.zeros(cols // (256 if q8k else 32) * (292 if q8k else 34), np.uint8)
        if q8k:
            orc.or_quantize_q8_k(pyoracle.ptr(x), pyoracle.ptr(q), cols, bits)
        else:
            orc.or_quantize_q8_0(pyoracle.ptr(x), pyoracle.ptr(q), cols)
        out.append(q)
    return np.concatenate(out)


@pytest.mark.parametrize("type_,rows,cols", [(Q4_0, 1024, 2048), (Q8_0, 300, 1024), (Q4_K, 512, 2048),
                                              (Q5_K, 512, 2048), (Q6_K, 256, 8192), (TQ2_0, 640, 2560),
                                              (Q4_K, 64, 9728)])  # rows wider than 8192: staged for n = 1 too
def test_noalloc_matmul_matches_matmul(lib, type_, rows, cols):
    orc = pyoracle.oracle_lib()
    be, _ = BLOCK[type_]
    w = synth.BLOCK_MAKERS[type_](rows * 31 + cols, rows * cols // be).reshape(-1)
    nbytes = lib.brisk_hip_packed_bytes(type_, rows, cols)
    wd = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    L.check(lib.brisk_hip_pack(type_, p(dev(w)), rows, cols, p(wd), None))
    flags = 1 if (type_ == TQ2_0 and rows % 16 == 0) else 0
    stride = rows + 5
    for n in ((67, 9) if cols <= 8192 else (9, 1)):  # the second call is smaller: nothing of the first may leak into it
        print(f"noalloc matmul: type {type_} {rows}x{cols} n={n}", flush=True)
        xd = dev(quantised_rows(orc, type_, rows, cols, n, 1000 + n))
        want = torch.full((n * stride,), -1.0, dtype=torch.float32, device="cuda")
        L.check(lib.brisk_hip_matmul(type_, flags, p(wd), rows, cols, p(xd), n, p(want), stride, None))
        got = torch.full((n * stride,), -2.0, dtype=torch.float32, device="cuda")
        L.check(lib.brisk_hip_matmul_noalloc(type_, flags, p(wd), rows, cols, p(xd), n, p(got), stride, None))
        torch.cuda.synchronize()
        g = got.cpu().numpy().reshape(n, stride)[:, :rows]
        e = want.cpu().numpy().reshape(n, stride)[:, :rows]
        np.testing.assert_array_equal(g.view(np.uint32), e.view(np.uint32))


def test_noalloc_matmul_refuses_oversized_batches(lib):
    rows, cols, n = 64, 8192, 400  # 400 x 8192 x 1.375 bytes > 4 MiB
    nbytes = lib.brisk_hip_packed_bytes(Q4_0, rows, cols)
    wd = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    xd = torch.zeros(n * cols // 32 * 34, dtype=torch.uint8, device="cuda")
    out = torch.zeros(n * rows, dtype=torch.float32, device="cuda")
    rc = lib.brisk_hip_matmul_noalloc(Q4_0, 0, p(wd), rows, cols, p(xd), n, p(out), rows, None)
    assert rc == -1
    assert b"no-alloc matmul holds 4194304" in lib.brisk_hip_last_error()
