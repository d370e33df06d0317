"""fp32 GEMM with direct HBM->LDS loads (every configuration of gemm_f32dma.hip,
selected with ORMI_GEMM_F32_DMA_CFG; the library reads it per call) through the
C-ABI: the four layouts, ragged M and N (clamped loads, guarded stores), a K
split with its finish pass, batched operands with a broadcast one, and the
in-kernel epilogue. Each result is checked against the float64 product within
the fp32 accumulation-order bound 2 K eps32 (|A| |B|); the same inputs through
the register-staged kernels (ORMI_GEMM_F32_DMA=0) meet the same bound.
"""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class GemmDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
                ("a", ctypes.c_void_p), ("a_stride_m", ctypes.c_int64), ("a_stride_k", ctypes.c_int64),
                ("b", ctypes.c_void_p), ("b_stride_k", ctypes.c_int64), ("b_stride_n", ctypes.c_int64),
                ("c", ctypes.c_void_p), ("batch_ndim", ctypes.c_int), ("batch_shape", ctypes.c_int * 4),
                ("a_batch_stride", ctypes.c_int64 * 4), ("b_batch_stride", ctypes.c_int64 * 4)]


class GemmEpilogue(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("fn", ctypes.c_int), ("form", ctypes.c_int), ("s", ctypes.c_void_p),
                ("d", ctypes.c_void_p), ("d_stride_m", ctypes.c_int64), ("d_stride_n", ctypes.c_int64),
                ("d_batch_stride", ctypes.c_int64 * 4), ("aux", ctypes.c_void_p)]


@pytest.fixture
def lib(cabi, hip):
    lib = cabi  # shared across test modules: no argtypes set here (byref needs none)
    saved = {k: os.environ.get(k) for k in ("ORMI_GEMM_F32_DMA", "ORMI_GEMM_F32_DMA_CFG")}
    bufs = []

    def dev(arr):
        arr = np.ascontiguousarray(arr, np.float32)
        p = ctypes.c_void_p()
        assert lib.ormi_hip_malloc(ctypes.byref(p), max(arr.nbytes, 4)) == 0
        if arr.nbytes:
            assert lib.ormi_hip_memcpy_h2d(p, arr.ctypes.data, arr.nbytes) == 0
        bufs.append(p)
        return p

    def read(p, shape):
        out = np.empty(shape, np.float32)
        assert lib.ormi_hip_synchronize() == 0
        assert lib.ormi_hip_memcpy_d2h(out.ctypes.data, p, out.nbytes) == 0
        return out

    lib.dev, lib.read = dev, read
    yield lib
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v
    for p in bufs:
        lib.ormi_hip_free(p)


def use(cfg):
    """cfg: a direct-load configuration id, or None for the register-staged kernels."""
    os.environ["ORMI_GEMM_F32_DMA"] = "0" if cfg is None else "1"
    os.environ["ORMI_GEMM_F32_DMA_CFG"] = "1" if cfg is None else str(cfg)


def bound(A, B):
    K = A.shape[-1]
    return 2 * K * np.finfo(np.float32).eps * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)) + 1e-30


def run(lib, A, B, layout, batch_b_broadcast=False):
    """C = A @ B (A (..., M, K), B (..., K, N)) with A / B stored transposed for 'T'."""
    batched = A.ndim == 3
    M, K = A.shape[-2:]
    N = B.shape[-1]
    a_host = A if layout[0] == "N" else np.swapaxes(A, -1, -2)
    b_host = B if layout[1] == "N" else np.swapaxes(B, -1, -2)
    if batch_b_broadcast:
        b_host = b_host[0]
    g = GemmDesc(dtype=0, M=M, N=N, K=K, a=lib.dev(a_host), b=lib.dev(b_host), c=lib.dev(np.zeros(A.shape[:-1] + (N,))))
    g.a_stride_m, g.a_stride_k = (K, 1) if layout[0] == "N" else (1, M)
    g.b_stride_k, g.b_stride_n = (N, 1) if layout[1] == "N" else (1, K)
    if batched:
        g.batch_ndim = 1
        g.batch_shape[0] = A.shape[0]
        g.a_batch_stride[0] = M * K
        g.b_batch_stride[0] = 0 if batch_b_broadcast else K * N
    assert lib.ormi_hip_gemm(ctypes.byref(g)) == 0, lib.ormi_hip_last_error()
    return lib.read(g.c, A.shape[:-1] + (N,))


# Shapes: whole tiles; ragged M and N with K in whole 32- and 64-deep tiles; a
# K of 96 (whole 32-deep tiles only: the 64-deep configurations fall back to
# the register-staged kernels); tiny.
SHAPES = [(256, 256, 128), (300, 520, 128), (96, 200, 192), (256, 512, 96), (4, 8, 64)]


@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, None])
@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
def test_direct_load_layouts_and_ragged_tiles(lib, cfg, layout):
    use(cfg)
    rng = np.random.default_rng(91)
    for M, N, K in SHAPES:
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((K, N)).astype(np.float32)
        err = np.abs(run(lib, A, B, layout) - A.astype(np.float64) @ B.astype(np.float64))
        assert np.all(err <= bound(A, B)), (cfg, layout, M, N, K, float(np.max(err / bound(A, B))))


@pytest.mark.parametrize("cfg", [1, 2, 4, 6, 7, 8, 9, None])
def test_direct_load_k_split_and_batches(lib, cfg):
    """One 128x128 tile over K = 4096 is split over the CUs (a finish pass sums
    the partials in split order); three batches against one broadcast B."""
    use(cfg)
    rng = np.random.default_rng(92)
    A = rng.standard_normal((128, 4096)).astype(np.float32)
    B = rng.standard_normal((4096, 128)).astype(np.float32)
    for layout in ("NN", "TN"):
        err = np.abs(run(lib, A, B, layout) - A.astype(np.float64) @ B.astype(np.float64))
        assert np.all(err <= bound(A, B)), (cfg, layout)
    A3 = rng.standard_normal((3, 256, 128)).astype(np.float32)
    B1 = rng.standard_normal((128, 384)).astype(np.float32)
    B3 = np.broadcast_to(B1, (3, 128, 384))
    for layout in ("NN", "NT"):
        got = run(lib, A3, B3, layout, batch_b_broadcast=True)
        want = A3.astype(np.float64) @ B1.astype(np.float64)
        assert np.all(np.abs(got - want) <= bound(A3, B3)), (cfg, layout)


@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9])
def test_direct_load_epilogue_in_kernel(lib, cfg):
    """C = D - s * (A @ B) (the SGD form) and C = relu(A @ B) with the product
    in aux, on a shape in whole tiles with no K split, so the epilogue runs in
    the kernel's store; bit-exact against the plain product of the same kernel
    followed by the same arithmetic in float32."""
    use(cfg)
    rng = np.random.default_rng(93)
    M, N, K = 512, 1024, 256
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    D = rng.standard_normal((M, N)).astype(np.float32)
    s = np.float32(0.01)
    plain = run(lib, A, B, "NN")
    g = GemmDesc(dtype=0, M=M, N=N, K=K, a=lib.dev(A), b=lib.dev(B), c=lib.dev(D.copy()))
    g.a_stride_m, g.a_stride_k, g.b_stride_k, g.b_stride_n = K, 1, N, 1
    e = GemmEpilogue(kind=1, form=1, s=lib.dev(np.array([s])), d=g.c, d_stride_m=N, d_stride_n=1)
    assert lib.ormi_hip_gemm_ex(ctypes.byref(g), ctypes.byref(e)) == 0, lib.ormi_hip_last_error()
    np.testing.assert_array_equal(lib.read(g.c, (M, N)), D - plain * s)  # in place: D is C
    aux = lib.dev(np.zeros((M, N)))
    g.c = lib.dev(np.zeros((M, N)))
    e = GemmEpilogue(kind=2, fn=1, aux=aux)
    assert lib.ormi_hip_gemm_ex(ctypes.byref(g), ctypes.byref(e)) == 0, lib.ormi_hip_last_error()
    np.testing.assert_array_equal(lib.read(aux, (M, N)), plain)
    np.testing.assert_array_equal(lib.read(g.c, (M, N)), np.maximum(plain, 0))


def _persist(on: bool):
    os.environ["ORMI_GEMM_PERSIST"] = "1" if on else "0"


# More whole 128x128 tiles than compute units: 512 tiles (a multiple of 8, the
# XCD-aware order), 289 (not a multiple of 8; some work-groups get 2 tiles,
# others 1), and 1024 (4 per work-group) with K = 64 (two k-tiles per tile:
# the stream crosses tiles inside the first loads).
PERSIST_SHAPES = [(2048, 4096, 256), (2176, 2176, 160), (4096, 4096, 64)]


@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
def test_persistent_kernel_matches_one_tile_kernel(lib, layout):
    """The persistent form runs each tile's MFMAs in the same order as the
    one-tile kernel, so the products are bit-identical; both stay within the
    fp32 bound of the float64 product."""
    use(1)
    rng = np.random.default_rng(94)
    try:
        for M, N, K in PERSIST_SHAPES:
            A = (rng.standard_normal((M, K)) / 8).astype(np.float32)
            B = (rng.standard_normal((K, N)) / 8).astype(np.float32)
            _persist(True)
            got = run(lib, A, B, layout)
            _persist(False)
            want = run(lib, A, B, layout)
            np.testing.assert_array_equal(got, want, err_msg=f"{layout} {M}x{N}x{K}")
            err = np.abs(got - A.astype(np.float64) @ B.astype(np.float64))
            assert np.all(err <= bound(A, B)), (layout, M, N, K)
    finally:
        os.environ.pop("ORMI_GEMM_PERSIST", None)


@pytest.mark.parametrize("kind", ["sgd", "gelu_aux", "gelu_grad"])
def test_persistent_kernel_epilogues_match_one_tile_kernel(lib, kind):
    """Epilogues in the persistent kernel's stores (the C5 weight gradient is
    the SGD form over 1024 tiles): bit-identical to the one-tile kernel's,
    D read in place for the SGD update."""
    use(1)
    rng = np.random.default_rng(95)
    M, N, K = 2048, 4096, 128
    A = (rng.standard_normal((M, K)) / 8).astype(np.float32)
    B = (rng.standard_normal((K, N)) / 8).astype(np.float32)
    D = rng.standard_normal((M, N)).astype(np.float32)
    s = lib.dev(np.array([1e-3], np.float32))
    outs = []
    try:
        for on in (True, False):
            # Activation epilogues take the persistent kernel only when asked (2).
            os.environ["ORMI_GEMM_PERSIST"] = "2" if on else "0"
            g = GemmDesc(dtype=0, M=M, N=N, K=K, a=lib.dev(A), b=lib.dev(B), c=lib.dev(D.copy()))
            g.a_stride_m, g.a_stride_k, g.b_stride_k, g.b_stride_n = K, 1, N, 1
            aux = None
            if kind == "sgd":
                e = GemmEpilogue(kind=1, form=1, s=s, d=g.c, d_stride_m=N, d_stride_n=1)
            elif kind == "gelu_aux":
                aux = lib.dev(np.zeros((M, N)))
                e = GemmEpilogue(kind=2, fn=7, aux=aux)
            else:
                e = GemmEpilogue(kind=3, fn=8, d=lib.dev(D), d_stride_m=N, d_stride_n=1)
            assert lib.ormi_hip_gemm_ex(ctypes.byref(g), ctypes.byref(e)) == 0, lib.ormi_hip_last_error()
            outs.append((lib.read(g.c, (M, N)), lib.read(aux, (M, N)) if aux is not None else None))
    finally:
        os.environ.pop("ORMI_GEMM_PERSIST", None)
    (c1, x1), (c0, x0) = outs
    np.testing.assert_array_equal(c1, c0)
    if x1 is not None:
        np.testing.assert_array_equal(x1, x0)
    assert np.all(np.isfinite(c1))
