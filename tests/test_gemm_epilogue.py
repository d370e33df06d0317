"""GEMM epilogue fusion: ormi_hip_gemm_ex and the HIP scheduler's matching of an
element-wise consumer of a matmul (SGD update, forward activation, activation
backward on the dX GEMM).

The bar is bit-exact against the unfused path (the same GEMM, then the
element-wise kernel): the epilogue rounds every operation on its own, as the
generated kernels do (no contraction), and calls the same device functions.
Against the CPU oracle: the fp32 pointwise tolerance (rtol 1e-6) on top of the
GEMM's accumulation-order bound 2 K eps32 (|A| |B|), scaled by the epilogue's
Lipschitz constant.
"""
import ctypes
import math
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["direct", "staged"])
def f32_kernels(request):
    """Every test runs on both fp32 GEMM families: the direct-load kernels (the
    default) and the register-staged ones (ORMI_GEMM_F32_DMA=0, read per call)."""
    old = os.environ.get("ORMI_GEMM_F32_DMA")
    os.environ["ORMI_GEMM_F32_DMA"] = "1" if request.param == "direct" else "0"
    yield request.param
    if old is None:
        os.environ.pop("ORMI_GEMM_F32_DMA", None)
    else:
        os.environ["ORMI_GEMM_F32_DMA"] = old


def T(data, dev, **kw):
    from ormi_amd import Tensor

    return Tensor(data, device=dev, **kw)


def bits_equal(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.dtype == b.dtype and a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def assert_near_oracle(got, ref, A, B, lip=1.0, scale=1.0):
    """|got - ref| <= lip * scale * 2 K eps32 (|A| |B|) + 1e-6 |ref| + 1e-7: the
    fp32 accumulation-order bound of the product, carried through an epilogue
    with Lipschitz constant lip and a scale factor."""
    K = A.shape[-1]
    bound = 2 * K * np.finfo(np.float32).eps * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    lim = lip * abs(scale) * bound + 1e-6 * np.abs(ref) + 1e-7
    assert np.all(err <= lim), f"max excess {np.max(err - lim):.3g}"


def fused_and_plain(ob, build):
    """build() -> list of Tensors to read. Run it with fusion on and off; return
    (fused arrays, plain arrays, epilogue GEMMs used by the fused run)."""
    ob.set_gemm_epilogue(True)
    c0 = ob.gemm_epilogue_count()
    fused = [t.numpy() for t in build()]
    used = ob.gemm_epilogue_count() - c0
    ob.set_gemm_epilogue(False)
    try:
        c1 = ob.gemm_epilogue_count()
        plain = [t.numpy() for t in build()]
        assert ob.gemm_epilogue_count() == c1
    finally:
        ob.set_gemm_epilogue(True)
    return fused, plain, used


# (M, K, N) -> dispatch (direct-load kernels / register-staged ones): the
# epilogue in the kernel's store (128x128 tiles / config 3); in the store (one
# tile / config 2); K split (finish pass); ragged tiles (finish pass);
# unaligned K (the generic kernel's store).
SHAPES = [(1024, 1024, 4096), (128, 64, 256), (256, 512, 512), (120, 64, 200), (100, 70, 130)]


def operands(seed, M, K, N):
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((M, K)).astype(np.float32) / math.sqrt(K)
    B = rng.standard_normal((K, N)).astype(np.float32)
    W = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal((N,)).astype(np.float32)
    return A, B, W, bias


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_scale_add_forms_fused_bit_exact(ob, hip, cpu, M, K, N):
    A, B, W, bias = operands(71, M, K, N)

    def build():
        a, b, w = T(A, hip), T(B, hip), T(W, hip)
        return [w - (a @ b) * 0.01,           # SGD form, D - p*s
                w + 0.25 * (a @ b),           # D + s*p
                (a @ b) * 3.0 - w,            # p*s - D
                (a @ b) + T(bias, hip),       # D broadcast along rows, no scale
                T(bias, hip) - (a @ b)]       # D - p
    fused, plain, used = fused_and_plain(ob, build)
    assert used == 5
    for f, p in zip(fused, plain):
        assert bits_equal(f, p)
    a, b, w = T(A, cpu), T(B, cpu), T(W, cpu)
    assert_near_oracle(fused[0], (w - (a @ b) * 0.01).numpy(), A, B, scale=0.01)
    assert_near_oracle(fused[3], ((a @ b) + T(bias, cpu)).numpy(), A, B)


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("act", ["relu", "tanh", "sigmoid", "gelu"])
def test_activation_epilogue_stores_product_too(ob, hip, cpu, M, K, N, act):
    A, B, _, _ = operands(72, M, K, N)
    keep = {}

    def build():
        p = T(A, hip) @ T(B, hip)
        y = getattr(p, act)()
        keep["p"] = p
        return [y, p]
    ob.set_gemm_epilogue(True)
    c0 = ob.gemm_epilogue_count()
    b = build()
    y_f = b[0].numpy()  # the activation first: the product rides along
    used = ob.gemm_epilogue_count() - c0
    p_f = b[1].numpy()
    assert used == 1
    assert ob.gemm_epilogue_count() - c0 == 1  # reading the product launched nothing new
    fused, plain, _ = fused_and_plain(ob, build)
    assert bits_equal(y_f, plain[0]) and bits_equal(p_f, plain[1])
    ref = getattr(T(A, cpu) @ T(B, cpu), act)().numpy()
    assert_near_oracle(y_f, ref, A, B, lip=1.13)  # max |gelu'| = 1.128...


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("act", ["relu", "gelu"])
def test_activation_backward_on_dx_gemm(ob, hip, cpu, M, K, N, act):
    """h.grad = (dz . W^T) * act'(h): MUL(MATMUL, STEP/GELU_GRAD(h))."""
    rng = np.random.default_rng(73)
    H = rng.standard_normal((M, K)).astype(np.float32)
    Wt = (rng.standard_normal((K, N)) / math.sqrt(K)).astype(np.float32)
    R = rng.standard_normal((M, N)).astype(np.float32)

    def run(dev):
        h = T(H, dev, requires_grad=True)
        z = getattr(h, act)() @ T(Wt, dev)
        (z * T(R, dev)).sum().backward()
        return [h.grad]
    fused, plain, used = fused_and_plain(ob, lambda: run(hip))
    assert used >= 1
    assert bits_equal(fused[0], plain[0])
    # grad = (R . Wt^T) * act'(h), |act'| <= 1.13
    assert_near_oracle(fused[0], run(cpu)[0].numpy(), R, Wt.T, lip=1.13)


def test_mul_by_operand_and_unmatched_forms(ob, hip):
    A, B, W, _ = operands(74, 256, 128, 256)

    def build():
        a, b, w = T(A, hip), T(B, hip), T(W, hip)
        p = a @ b
        return [p * w,                 # p * D: identity function
                (a @ b) * (w * 2.0),   # D is element-wise: not matched, plain path
                ((a @ b) * 2.0).exp()] # not an epilogue form
    fused, plain, used = fused_and_plain(ob, build)
    assert used == 1
    for f, p in zip(fused, plain):
        assert bits_equal(f, p)


def test_realized_product_is_not_recomputed(ob, hip):
    A, B, W, _ = operands(75, 128, 64, 256)
    a, b, w = T(A, hip), T(B, hip), T(W, hip)
    p = (a @ b).realize()
    c0 = ob.gemm_epilogue_count()
    out = (w - p * 0.5).numpy()
    assert ob.gemm_epilogue_count() == c0
    assert bits_equal(out, (W - (p.numpy() * np.float32(0.5))).astype(np.float32))


def mlp_step(dev, X, Yt, Ws, lr=1e-3):
    ws = [T(w, dev, requires_grad=True) for w in Ws]
    h = T(X, dev)
    for i, w in enumerate(ws):
        h = h @ w
        if i < len(ws) - 1:
            h = h.gelu()
    d = h - T(Yt, dev)
    loss = (d * d).sum() * (1.0 / (X.shape[0] * Yt.shape[1]))
    loss.backward()
    new = [(w - w.grad * lr) for w in ws]
    return [loss] + new


def test_mlp_step_fused_equals_unfused(ob, hip, cpu):
    """The C5 step shape in miniature: forward GELUs, dGELU on the dX GEMMs and
    the three SGD updates all run as epilogues, bit-exact with the unfused step."""
    rng = np.random.default_rng(4)
    dims = [256, 1024, 1024, 256]
    X = rng.normal(0, 1, (256, dims[0])).astype(np.float32)
    Yt = rng.normal(0, 1, (256, dims[-1])).astype(np.float32)
    Ws = [rng.uniform(-math.sqrt(6 / i), math.sqrt(6 / i), (i, o)).astype(np.float32) for i, o in zip(dims, dims[1:])]
    fused, plain, used = fused_and_plain(ob, lambda: mlp_step(hip, X, Yt, Ws))
    assert used >= 7  # 2 GELU + 2 dGELU + 3 SGD
    for f, p in zip(fused, plain):
        assert bits_equal(f, p)
    # Against the oracle: accumulation-order differences over K = 1024 through
    # three layers and back (the tight-tolerance MLP parity test runs the same
    # fused path at K <= 256).
    ref = [t.numpy() for t in mlp_step(cpu, X, Yt, Ws)]
    np.testing.assert_allclose(fused[0], ref[0], rtol=1e-4)
    for f, r in zip(fused[1:], ref[1:]):
        np.testing.assert_allclose(f, r, rtol=1e-4, atol=1e-5)


def test_mlp_step_updates_first_fuses_forward_gelu(ob, hip):
    """Realizing the weight updates before the loss (as a training loop that
    only reads the new weights does) reaches each hidden product first through
    the backward's gelu'(p). The product still runs as its forward GELU's GEMM
    epilogue, storing p and gelu(p) together: 2 GELU + 2 dGELU + 3 SGD epilogues,
    bit-exact with the unfused step."""
    rng = np.random.default_rng(5)
    dims = [256, 512, 512, 256]
    X = rng.normal(0, 1, (128, dims[0])).astype(np.float32)
    Yt = rng.normal(0, 1, (128, dims[-1])).astype(np.float32)
    Ws = [rng.uniform(-math.sqrt(6 / i), math.sqrt(6 / i), (i, o)).astype(np.float32) for i, o in zip(dims, dims[1:])]

    def updates_first():
        out = mlp_step(hip, X, Yt, Ws)
        return out[1:] + out[:1]

    fused, plain, used = fused_and_plain(ob, updates_first)
    assert used >= 7, used
    for f, p in zip(fused, plain):
        assert bits_equal(f, p)


# ------------------------------------------------------------- the C ABI --
class Desc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
                ("a", ctypes.c_void_p), ("a_stride_m", ctypes.c_int64), ("a_stride_k", ctypes.c_int64),
                ("b", ctypes.c_void_p), ("b_stride_k", ctypes.c_int64), ("b_stride_n", ctypes.c_int64),
                ("c", ctypes.c_void_p), ("batch_ndim", ctypes.c_int), ("batch_shape", ctypes.c_int * 4),
                ("a_batch_stride", ctypes.c_int64 * 4), ("b_batch_stride", ctypes.c_int64 * 4)]


class Epi(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("fn", ctypes.c_int), ("form", ctypes.c_int), ("s", ctypes.c_void_p),
                ("d", ctypes.c_void_p), ("d_stride_m", ctypes.c_int64), ("d_stride_n", ctypes.c_int64),
                ("d_batch_stride", ctypes.c_int64 * 4), ("aux", ctypes.c_void_p)]


class Dev:
    def __init__(self, lib):
        self.lib, self.ptrs = lib, []

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = ctypes.c_void_p()
        assert self.lib.ormi_hip_malloc(ctypes.byref(p), max(arr.nbytes, 4)) == 0
        assert self.lib.ormi_hip_memcpy_h2d(p, arr.ctypes.data, arr.nbytes) == 0
        self.ptrs.append(p)
        return p

    def get(self, p, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        assert self.lib.ormi_hip_synchronize() == 0
        assert self.lib.ormi_hip_memcpy_d2h(out.ctypes.data, p, out.nbytes) == 0
        return out

    def free(self):
        for p in self.ptrs:
            self.lib.ormi_hip_free(p)


def bf16_bits(x):
    u = x.astype(np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("dtype,M,K,N,batch", [(0, 256, 512, 256, 1), (0, 96, 64, 128, 3), (3, 256, 256, 256, 1),
                                               (3, 64, 96, 128, 2), (0, 64, 0, 64, 1)])
def test_cabi_add_in_place_and_batched(cabi, dtype, M, K, N, batch):
    """C = C - (A B) * s with D == C (in place), batched (broadcast B), fp32 and
    bf16 (its kernels take the finish pass), and K = 0 (the product is 0)."""
    rng = np.random.default_rng(76)
    A = rng.standard_normal((batch, M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    W = rng.standard_normal((batch, M, N)).astype(np.float32)
    s = np.array(0.125, np.float32)
    dev = Dev(cabi)
    try:
        if dtype == 3:
            pa, pb = dev.put(bf16_bits(A)), dev.put(bf16_bits(B))
        else:
            pa, pb = dev.put(A), dev.put(B)
        pc, pp, ps = dev.put(W), dev.put(np.zeros((batch, M, N), np.float32)), dev.put(s)
        d = Desc(dtype=dtype, M=M, N=N, K=K, a=pa, a_stride_m=K, a_stride_k=1, b=pb, b_stride_k=N, b_stride_n=1, c=pp)
        if batch > 1:
            d.batch_ndim, d.batch_shape[0], d.a_batch_stride[0], d.b_batch_stride[0] = 1, batch, M * K, 0
        assert cabi.ormi_hip_gemm(ctypes.byref(d)) == 0, cabi.ormi_hip_last_error()
        P = dev.get(pp, (batch, M, N))
        d.c = pc
        e = Epi(kind=1, fn=0, form=1, s=ps, d=pc, d_stride_m=N, d_stride_n=1)
        e.d_batch_stride[0] = M * N
        assert cabi.ormi_hip_gemm_ex(ctypes.byref(d), ctypes.byref(e)) == 0, cabi.ormi_hip_last_error()
        got = dev.get(pc, (batch, M, N))
        assert bits_equal(got, (W - (P * s).astype(np.float32)).astype(np.float32))
    finally:
        dev.free()


def test_cabi_unary_aux_on_k_split(cabi):
    """gelu epilogue with aux through the finish pass of a K split."""
    rng = np.random.default_rng(77)
    M, K, N = 128, 4096, 256  # 1 tile: K is split
    A = (rng.standard_normal((M, K)) / 64).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    dev = Dev(cabi)
    try:
        pa, pb = dev.put(A), dev.put(B)
        pp, pc, px = (dev.put(np.zeros((M, N), np.float32)) for _ in range(3))
        d = Desc(dtype=0, M=M, N=N, K=K, a=pa, a_stride_m=K, a_stride_k=1, b=pb, b_stride_k=N, b_stride_n=1, c=pp)
        assert cabi.ormi_hip_gemm(ctypes.byref(d)) == 0
        d.c = pc
        e = Epi(kind=2, fn=7, aux=px)
        assert cabi.ormi_hip_gemm_ex(ctypes.byref(d), ctypes.byref(e)) == 0, cabi.ormi_hip_last_error()
        P, Y, X = dev.get(pp, (M, N)), dev.get(pc, (M, N)), dev.get(px, (M, N))
        assert bits_equal(X, P)
        ref = 0.5 * P.astype(np.float64) * (1 + np.vectorize(math.erf)(P.astype(np.float64) / math.sqrt(2)))
        np.testing.assert_allclose(Y, ref, rtol=1e-6, atol=1e-6)
    finally:
        dev.free()
