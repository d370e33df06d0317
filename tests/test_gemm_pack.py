"""GEMMs whose operands the direct-load kernels cannot take as given, through
the C-ABI: a unit-stride extent or another stride not in whole 16-byte chunks
(odd N, odd K, odd leading dimensions), no unit stride at all, or K not in
whole tiles. Such operands are packed into dense k-contiguous buffers,
zero-padded along K to a multiple of 64, and the product runs on the
direct-load MFMA kernels (ORMI_GEMM_PACK=0 keeps the generic or
register-staged kernel instead). Each result is checked against the float64
product of the operand values within 2 K eps32 (|A| |B|), on both paths, with
batches (one operand broadcast) and an epilogue in the finish pass."""
import ctypes
import os

import numpy as np
import pytest

from test_gemm_f32dma import GemmDesc, GemmEpilogue
from test_gemm_16bit_cfgs import BF16, F16, to_16

pytestmark = pytest.mark.gpu

F32 = 0


@pytest.fixture
def lib(cabi, hip):
    lib = cabi
    saved = os.environ.get("ORMI_GEMM_PACK")
    bufs = []

    def dev(arr):
        arr = np.ascontiguousarray(arr)
        p = ctypes.c_void_p()
        assert lib.ormi_hip_malloc(ctypes.byref(p), max(arr.nbytes, 4)) == 0
        assert lib.ormi_hip_memcpy_h2d(p, arr.ctypes.data, arr.nbytes) == 0
        bufs.append(p)
        return p

    lib.dev = dev
    yield lib
    if saved is None:
        os.environ.pop("ORMI_GEMM_PACK", None)
    else:
        os.environ["ORMI_GEMM_PACK"] = saved
    for p in bufs:
        lib.ormi_hip_free(p)


def host(x, dt):
    """Device bits and exact float64 values of x in dtype dt."""
    if dt == F32:
        x = np.ascontiguousarray(x, np.float32)
        return x, x.astype(np.float64)
    return to_16(x, dt)


def run(lib, dt, a_mem, b_mem, M, N, K, a_st, b_st, pack, batch=None, epi=None, out=None):
    """C = A @ B from operand memories with element strides a_st = (m, k),
    b_st = (k, n); batch = (count, a batch stride, b batch stride)."""
    os.environ["ORMI_GEMM_PACK"] = "1" if pack else "0"
    rows = (batch[0] if batch else 1) * M
    c = out if out is not None else lib.dev(np.full((rows, N), np.nan, np.float32))
    g = GemmDesc(dtype=dt, M=M, N=N, K=K, a=lib.dev(a_mem), b=lib.dev(b_mem), c=c)
    g.a_stride_m, g.a_stride_k = a_st
    g.b_stride_k, g.b_stride_n = b_st
    if batch:
        g.batch_ndim = 1
        g.batch_shape[0], g.a_batch_stride[0], g.b_batch_stride[0] = batch
    if epi is None:
        assert lib.ormi_hip_gemm(ctypes.byref(g)) == 0, lib.ormi_hip_last_error()
    else:
        assert lib.ormi_hip_gemm_ex(ctypes.byref(g), ctypes.byref(epi)) == 0, lib.ormi_hip_last_error()
    res = np.empty((rows, N), np.float32)
    assert lib.ormi_hip_synchronize() == 0
    assert lib.ormi_hip_memcpy_d2h(res.ctypes.data, c, res.nbytes) == 0
    return res


def bound(a64, b64, K):
    return 2 * K * np.finfo(np.float32).eps * (np.abs(a64) @ np.abs(b64))


# (M, N, K, layout of A, layout of B): N = element stride pattern of the operand
# memory. "N": A (M, K) row-major, B (K, N) row-major; "T": stored transposed;
# "P": padded leading dimension of odd length (ld = extent + 3).
CASES = [
    (260, 257, 264, "N", "N"),    # odd N: B's rows are not whole 16-byte chunks
    (257, 264, 260, "N", "T"),    # odd M, K = 260 (not a multiple of 32)
    (264, 258, 251, "T", "N"),    # odd K, both operands stored with odd rows
    (250, 262, 270, "P", "P"),    # odd leading dimensions on both operands
    (300, 300, 300, "T", "T"),
]


def memory(x, layout, rng):
    """Operand x (rows, cols) in memory as the layout says, with its element strides (row, col)."""
    r, c = x.shape
    if layout == "N":
        return x, (c, 1)
    if layout == "T":
        return np.ascontiguousarray(x.T), (1, r)
    ld = c + 3
    mem = np.zeros((r, ld), x.dtype)
    mem[:, :c] = x
    return mem, (ld, 1)


@pytest.mark.parametrize("dt", [F32, BF16, F16])
def test_packed_operands_match_float64(lib, dt):
    rng = np.random.default_rng(151 + dt)
    for M, N, K, la, lb in CASES:
        assert M * N * K >= 1 << 24  # large enough to take the packed path
        a_bits, a64 = host(rng.standard_normal((M, K)) / 8, dt)
        b_bits, b64 = host(rng.standard_normal((K, N)) / 8, dt)
        a_mem, (a_r, a_c) = memory(a_bits, la, rng)
        b_mem, (b_r, b_c) = memory(b_bits, lb, rng)
        want, bd = a64 @ b64, bound(a64, b64, K)
        for pack in (True, False):
            got = run(lib, dt, a_mem, b_mem, M, N, K, (a_r, a_c), (b_r, b_c), pack)
            assert np.all(np.abs(got - want) <= bd), (dt, M, N, K, la, lb, pack)


def test_packed_batches_with_broadcast_and_epilogue(lib):
    """Three batches of an odd-N product against one broadcast B, then the SGD
    epilogue C = D - s (A @ B) in the finish pass."""
    rng = np.random.default_rng(157)
    nb, M, N, K = 3, 256, 257, 272
    a_bits, a64 = host(rng.standard_normal((nb * M, K)) / 8, BF16)
    b_bits, b64 = host(rng.standard_normal((K, N)) / 8, BF16)
    want = a64 @ b64
    bd = bound(a64, b64, K)
    for pack in (True, False):
        got = run(lib, BF16, a_bits, b_bits, M, N, K, (K, 1), (N, 1), pack, batch=(nb, M * K, 0))
        assert np.all(np.abs(got - want) <= bd), pack
    D = rng.standard_normal((nb * M, N)).astype(np.float32)
    s = lib.dev(np.array([0.01], np.float32))
    c = lib.dev(D)
    e = GemmEpilogue(kind=1, form=1, s=s, d=c, d_stride_m=N, d_stride_n=1)
    e.d_batch_stride[0] = M * N
    got = run(lib, BF16, a_bits, b_bits, M, N, K, (K, 1), (N, 1), True, batch=(nb, M * K, 0), epi=e, out=c)
    prod = run(lib, BF16, a_bits, b_bits, M, N, K, (K, 1), (N, 1), True, batch=(nb, M * K, 0))
    np.testing.assert_array_equal(got, D - prod * np.float32(0.01))


def test_large_product_with_k_not_in_whole_tiles_is_packed(lib):
    """An fp32 product of 2^32 multiply-adds or more whose K (4100) is not a
    multiple of the direct-load depth: packed to K 4160 and run on the
    direct-load kernel instead of the register-staged one."""
    rng = np.random.default_rng(159)
    M, N, K = 1024, 1024, 4100
    assert M * N * K >= 1 << 32
    a_bits, a64 = host(rng.standard_normal((M, K)) / 8, F32)
    b_bits, b64 = host(rng.standard_normal((K, N)) / 8, F32)
    want, bd = a64 @ b64, bound(a64, b64, K)
    for pack in (True, False):
        got = run(lib, F32, a_bits, b_bits, M, N, K, (K, 1), (N, 1), pack)
        assert np.all(np.abs(got - want) <= bd), pack
