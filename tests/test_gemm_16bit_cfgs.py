"""16-bit GEMM configurations through the C-ABI (ORMI_GEMM_DMA_CFG, read per
call): the whole-line kernel for a k-contiguous A (configurations 12 and 15,
256x256 and 128x128 tiles, the defaults for NN and NT with K a multiple of 64)
against the interleaved half-line kernel of the same tile (9 and 13). Both run the same MFMAs in the same order,
so with the same K split (none: ORMI_GEMM_MAX_SPLITS=1; the two kernels'
depths, 64 and 32, would otherwise choose different splits for some shapes)
their outputs must be bit-identical. Each result, the default's with its own K
split included, is checked against the float64 product of the bf16 / fp16
values within 2 K eps32 (|A| |B|). Covers the four layouts, ragged M and N,
K = 64 (one pair of k-tiles), an odd number of pairs, a long K with and
without a split, and batches against a broadcast B."""
import ctypes
import os

import numpy as np
import pytest

from test_gemm_f32dma import GemmDesc

pytestmark = pytest.mark.gpu

BF16, F16 = 3, 4  # ORMI_DTYPE_BF16, ORMI_DTYPE_F16 (include/ormi_hip.h)


def to_16(x: np.ndarray, dt: int):
    """Host bits and exact float64 values of x rounded to bf16 / fp16 (nearest even)."""
    x = np.ascontiguousarray(x, np.float32)
    if dt == F16:
        h = x.astype(np.float16)
        return h.view(np.uint16), h.astype(np.float64)
    u = x.view(np.uint32).astype(np.uint64)
    bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return bits, (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.fixture
def lib(cabi, hip):
    lib = cabi
    saved = {k: os.environ.get(k) for k in ("ORMI_GEMM_DMA_CFG", "ORMI_GEMM_MAX_SPLITS")}
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
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v
    for p in bufs:
        lib.ormi_hip_free(p)


def gemm(lib, cfg, dt, a_bits, b_bits, M, N, K, layout, batch=0, split=True):
    """C (fp32) = A @ B from 16-bit host bits stored as the layout says (T =
    transposed); cfg None is the default configuration, split=False forbids a
    K split."""
    for key, val in (("ORMI_GEMM_DMA_CFG", cfg), ("ORMI_GEMM_MAX_SPLITS", None if split else 1)):
        if val is None:
            os.environ.pop(key, None)
        else:
            os.environ[key] = str(val)
    rows = max(batch, 1) * M
    c = lib.dev(np.full((rows, N), np.nan, np.float32))
    g = GemmDesc(dtype=dt, M=M, N=N, K=K, a=lib.dev(a_bits), b=lib.dev(b_bits), c=c)
    g.a_stride_m, g.a_stride_k = (K, 1) if layout[0] == "N" else (1, M)
    g.b_stride_k, g.b_stride_n = (N, 1) if layout[1] == "N" else (1, K)
    if batch:
        g.batch_ndim = 1
        g.batch_shape[0] = batch
        g.a_batch_stride[0] = M * K
        g.b_batch_stride[0] = 0  # one B for every batch
    assert lib.ormi_hip_gemm(ctypes.byref(g)) == 0, lib.ormi_hip_last_error()
    out = np.empty((rows, N), np.float32)
    assert lib.ormi_hip_synchronize() == 0
    assert lib.ormi_hip_memcpy_d2h(out.ctypes.data, c, out.nbytes) == 0
    return out


# (M, N, K): whole tiles; ragged M and N; one pair of k-tiles; an odd number of
# pairs; a long K that the two tiles split across the compute units.
SHAPES = [(512, 256, 256), (300, 136, 192), (264, 520, 64), (256, 256, 320), (264, 136, 4096)]


@pytest.mark.parametrize("dt", [BF16, F16])
@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
def test_whole_line_kernel_matches_interleaved_bit_for_bit(lib, dt, layout):
    rng = np.random.default_rng(131 + dt)
    for M, N, K in SHAPES:
        a_bits, a64 = to_16(rng.standard_normal((M, K)) / 8, dt)
        b_bits, b64 = to_16(rng.standard_normal((K, N)) / 8, dt)
        a_store = a_bits if layout[0] == "N" else np.ascontiguousarray(a_bits.T)
        b_store = b_bits if layout[1] == "N" else np.ascontiguousarray(b_bits.T)
        want = a64 @ b64
        bound = 2 * K * np.finfo(np.float32).eps * (np.abs(a64) @ np.abs(b64))
        # (interleaved, whole-line) pairs: 256x256 tiles (9, 12), 128x128 (13, 15).
        for half, whole in ((9, 12), (13, 15)):
            got_h = gemm(lib, half, dt, a_store, b_store, M, N, K, layout, split=False)
            got_w = gemm(lib, whole, dt, a_store, b_store, M, N, K, layout, split=False)
            assert np.all(np.abs(got_h - want) <= bound), (half, layout, M, N, K)
            assert np.array_equal(got_w, got_h), (whole, layout, M, N, K)
        got = gemm(lib, None, dt, a_store, b_store, M, N, K, layout)
        assert np.all(np.abs(got - want) <= bound), (layout, M, N, K)


@pytest.mark.parametrize("layout", ["NN", "NT"])
def test_whole_line_kernel_batches_with_broadcast_b(lib, layout):
    rng = np.random.default_rng(137)
    batch, M, N, K = 3, 256, 384, 128
    a_bits, a64 = to_16(rng.standard_normal((batch * M, K)) / 8, BF16)
    b_bits, b64 = to_16(rng.standard_normal((K, N)) / 8, BF16)
    a_store = a_bits if layout[0] == "N" else None
    b_store = b_bits if layout[1] == "N" else np.ascontiguousarray(b_bits.T)
    want = a64 @ b64
    bound = 2 * K * np.finfo(np.float32).eps * (np.abs(a64) @ np.abs(b64))
    for half, whole in ((9, 12), (13, 15)):
        got_w = gemm(lib, whole, BF16, a_store, b_store, M, N, K, layout, batch=batch, split=False)
        got_h = gemm(lib, half, BF16, a_store, b_store, M, N, K, layout, batch=batch, split=False)
        assert np.all(np.abs(got_w - want) <= bound), whole
        assert np.array_equal(got_w, got_h), whole


# Tile counts T = tiles_m * tiles_n (256x256 tiles) that are multiples of 8, so
# the XCD remap (t -> (t & 7) * T/8 + t/8) runs, with tiles_m not a multiple of
# the 4-row tile group, so the last group is ragged: 4x8 = 32 (no ragged group),
# 6x4 = 24 with a ragged M, 5x8 = 40 with a ragged N and an odd number of k-tile
# pairs, 3x8 = 24 with one pair.
REMAP_SHAPES = [(1024, 2048, 128), (1400, 1024, 128), (1280, 1896, 192), (700, 2048, 64)]


@pytest.mark.parametrize("layout", ["NN", "NT"])
def test_whole_line_kernel_xcd_remap_and_ragged_groups(lib, layout):
    """Configuration 12 (the default for 256 or more 256x256 tiles, C4 4096^3
    included) against 9 where the tile remap and a ragged tile group apply:
    bit for bit, and within 2 K eps32 (|A| |B|) of the float64 product."""
    rng = np.random.default_rng(139)
    for M, N, K in REMAP_SHAPES:
        tiles = ((M + 255) // 256) * ((N + 255) // 256)
        assert tiles % 8 == 0
        a_bits, a64 = to_16(rng.standard_normal((M, K)) / 8, BF16)
        b_bits, b64 = to_16(rng.standard_normal((K, N)) / 8, BF16)
        b_store = b_bits if layout[1] == "N" else np.ascontiguousarray(b_bits.T)
        want = a64 @ b64
        bound = 2 * K * np.finfo(np.float32).eps * (np.abs(a64) @ np.abs(b64))
        got_h = gemm(lib, 9, BF16, a_bits, b_store, M, N, K, layout, split=False)
        got_w = gemm(lib, 12, BF16, a_bits, b_store, M, N, K, layout, split=False)
        assert np.all(np.abs(got_w - want) <= bound), (layout, M, N, K)
        assert np.array_equal(got_w, got_h), (layout, M, N, K)
