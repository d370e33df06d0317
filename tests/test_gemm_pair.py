"""ormi_hip_gemm_pair: two independent products as one call, the backward of a
MATMUL (dX = dZ Y^T and dY = X^T dZ on one dZ, reference
csrc/core/ops/blas/matmul.cpp:84-124, each a separate cuda::matmul there).

The pair kernel computes every tile with the same k-steps, in the same order,
and the same store epilogue as the product's own launch, so its outputs are
compared BIT FOR BIT with ormi_hip_gemm_ex on each descriptor in turn, over:
  * the epilogue pairs it is built for (plain, the activation's derivative on
    dX, the SGD update in place on dW) and the C5 step's shapes;
  * tile counts that are not multiples of the work-group count or of 8 (some
    work-groups take more tiles, the XCD order does not apply), products of
    different depth (the stream changes k-tile count where it changes product),
    and either product first in the call;
and the calls that must NOT group (a product with fewer tiles than compute
units, one product reading the other's output, an activation epilogue,
layouts the kernel is not built for, ORMI_GEMM_PAIR=0, and by default a pair
deeper than 64 k-tiles per work-group, such as C5's layer 2): those run as two calls
in order, which for the dependent pair means the second reads the first's
result. ORMI_GEMM_PAIR=2 groups the deep pairs too, which is how the kernel is
checked at C5's shapes. An invalid descriptor launches nothing. The products themselves are
checked against float64 elsewhere (tests/test_gemm_f32dma.py); here a sample of
rows is, as a guard against two equally wrong paths.
"""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NONE, ADD, UNARY, MUL_FN_D = 0, 1, 2, 3
GELU, GELU_GRAD = 7, 8


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


class Dev:
    def __init__(self, lib):
        self.lib, self.bufs = lib, []

    def put(self, arr):
        arr = np.ascontiguousarray(arr, np.float32)
        p = ctypes.c_void_p()
        assert self.lib.ormi_hip_malloc(ctypes.byref(p), max(arr.nbytes, 4)) == 0
        assert self.lib.ormi_hip_memcpy_h2d(p, arr.ctypes.data, arr.nbytes) == 0
        self.bufs.append(p)
        return p

    def get(self, p, shape):
        out = np.empty(shape, np.float32)
        assert self.lib.ormi_hip_synchronize() == 0
        assert self.lib.ormi_hip_memcpy_d2h(out.ctypes.data, p, out.nbytes) == 0
        return out

    def free(self):
        for p in self.bufs:
            self.lib.ormi_hip_free(p)
        self.bufs = []


@pytest.fixture
def dev(cabi, hip):
    cabi.ormi_hip_gemm_pair.argtypes = [ctypes.c_void_p] * 4 + [ctypes.POINTER(ctypes.c_int)]
    saved = {k: os.environ.get(k) for k in ("ORMI_GEMM_PAIR", "ORMI_GEMM_F32_DMA", "ORMI_GEMM_F32_DMA_CFG")}
    for k in saved:
        os.environ.pop(k, None)
    d = Dev(cabi)
    os.environ["ORMI_GEMM_PAIR"] = "2"  # group whatever the depth; tests of the default set it back
    yield d
    d.free()
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


class Problem:
    """One product on the device with its epilogue: the dX form (A = dZ [M, K]
    row-major, B = W^T as a view of W [N, K]: both k-contiguous) or the dW form
    (A = X^T as a view of X [K, M], B = dZ [K, N]: both mn-contiguous), or
    plain row-major NN."""

    def __init__(self, dev, rng, form, M, N, K, epi=NONE, c_init=None):
        self.M, self.N, self.K, self.form = M, N, K, form
        A = (rng.standard_normal((M, K)) / 8).astype(np.float32)
        B = (rng.standard_normal((K, N)) / 8).astype(np.float32)
        self.A, self.B = A, B
        d = GemmDesc(dtype=0, M=M, N=N, K=K)
        if form == "dx":
            d.a, d.a_stride_m, d.a_stride_k = dev.put(A), K, 1
            d.b, d.b_stride_k, d.b_stride_n = dev.put(B.T.copy()), 1, K
        elif form == "dw":
            d.a, d.a_stride_m, d.a_stride_k = dev.put(A.T.copy()), 1, M
            d.b, d.b_stride_k, d.b_stride_n = dev.put(B), N, 1
        else:
            d.a, d.a_stride_m, d.a_stride_k = dev.put(A), K, 1
            d.b, d.b_stride_k, d.b_stride_n = dev.put(B), N, 1
        self.c0 = (rng.standard_normal((M, N)).astype(np.float32) if c_init is None else c_init)
        d.c = dev.put(self.c0)
        self.desc = d
        e = GemmEpilogue(kind=epi)
        if epi == MUL_FN_D:
            e.fn, e.d, e.d_stride_m, e.d_stride_n = GELU_GRAD, dev.put(rng.standard_normal((M, N))), N, 1
        elif epi == ADD:  # W - grad * lr, in place on C
            e.form, e.s, e.d, e.d_stride_m, e.d_stride_n = 1, dev.put(np.array([1e-3], np.float32)), d.c, N, 1
        elif epi == UNARY:
            e.fn, e.aux = GELU, dev.put(np.zeros((M, N), np.float32))
        self.epi = e
        self.dev = dev

    def reset(self):
        assert self.dev.lib.ormi_hip_memcpy_h2d(self.desc.c, self.c0.ctypes.data, self.c0.nbytes) == 0

    def result(self):
        return self.dev.get(self.desc.c, (self.M, self.N))


def run_pair(dev, p0, p1):
    grouped = ctypes.c_int(-1)
    rc = dev.lib.ormi_hip_gemm_pair(ctypes.byref(p0.desc), ctypes.byref(p0.epi), ctypes.byref(p1.desc),
                                    ctypes.byref(p1.epi), ctypes.byref(grouped))
    assert rc == 0, dev.lib.ormi_hip_last_error()
    return grouped.value


def run_each(dev, *ps):
    for p in ps:
        assert dev.lib.ormi_hip_gemm_ex(ctypes.byref(p.desc), ctypes.byref(p.epi)) == 0, dev.lib.ormi_hip_last_error()


def pair_vs_each(dev, p0, p1):
    """(grouped flag, [pair results], [one-call results]); each product's C is
    reset to its initial contents before each run (the SGD form updates C)."""
    p0.reset(), p1.reset()
    g = run_pair(dev, p0, p1)
    got = [p0.result(), p1.result()]
    p0.reset(), p1.reset()
    run_each(dev, p0, p1)
    want = [p0.result(), p1.result()]
    return g, got, want


def check_rows(p, got, rows=8):
    """A sample of rows against float64 (plain products only)."""
    if p.epi.kind != NONE:
        return
    idx = np.linspace(0, p.M - 1, rows).astype(int)
    ref = p.A[idx].astype(np.float64) @ p.B.astype(np.float64)
    bound = 2 * p.K * np.finfo(np.float32).eps * (np.abs(p.A[idx]).astype(np.float64) @ np.abs(p.B).astype(np.float64))
    assert np.all(np.abs(got[idx] - ref) <= bound + 1e-30)


EPIS = [(NONE, NONE), (MUL_FN_D, NONE), (NONE, ADD), (MUL_FN_D, ADD)]


@pytest.mark.parametrize("e0,e1", EPIS)
def test_c5_layer3_pair_is_bit_identical_to_two_calls(dev, e0, e1):
    """dX = dY W3^T (1024 x 4096, K 1024) and dW3 = H2^T dY (4096 x 1024, K 1024):
    256 tiles each, two per work-group (grouped on request: 64 k-tiles per
    work-group)."""
    rng = np.random.default_rng(100 + 4 * e0 + e1)
    p0 = Problem(dev, rng, "dx", 1024, 4096, 1024, e0)
    p1 = Problem(dev, rng, "dw", 4096, 1024, 1024, e1)
    g, got, want = pair_vs_each(dev, p0, p1)
    assert g == 1
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)
    check_rows(p0, got[0])
    check_rows(p1, got[1])


def test_c5_layer2_pair_is_bit_identical_to_two_calls(dev):
    """dZ1 = (dZ2 W2^T) gelu'(Z1) (1024 x 4096, K 4096: 256 tiles of 128
    k-tiles) and W2 - lr H1^T dZ2 (4096 x 4096, K 1024: 1024 tiles of 32):
    each work-group streams one deep tile, then four shallow ones."""
    rng = np.random.default_rng(7)
    p0 = Problem(dev, rng, "dx", 1024, 4096, 4096, MUL_FN_D)
    p1 = Problem(dev, rng, "dw", 4096, 4096, 1024, ADD)
    g, got, want = pair_vs_each(dev, p0, p1)
    assert g == 1
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)


# (M0, N0, K0, M1, N1, K1): 289 + 256 tiles (neither a multiple of the other,
# 289 not of 8), 256 + 289, 300 + 512 (300 = 12 x 25), depths 96, 160, 32, 64.
UNEVEN = [(2176, 2176, 96, 2048, 2048, 160), (2048, 2048, 32, 2176, 2176, 64), (1536, 3200, 64, 2048, 4096, 32)]


@pytest.mark.parametrize("shape", UNEVEN)
@pytest.mark.parametrize("order", ["dx_first", "dw_first"])
def test_uneven_tile_counts_and_either_order(dev, shape, order):
    M0, N0, K0, M1, N1, K1 = shape
    rng = np.random.default_rng(M0 + N1 + K0)
    px = Problem(dev, rng, "dx", M0, N0, K0, MUL_FN_D)
    pw = Problem(dev, rng, "dw", M1, N1, K1, NONE)
    p0, p1 = (px, pw) if order == "dx_first" else (pw, px)
    g, got, want = pair_vs_each(dev, p0, p1)
    assert g == 1
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)
    check_rows(pw, got[0] if pw is p0 else got[1])


@pytest.mark.parametrize("K,grouped", [(256, 1), (1024, 1), (2048, 0)])
def test_default_groups_shallow_pairs_only(dev, K, grouped):
    """ORMI_GEMM_PAIR unset: the C5 layer-3 shapes at depth K group while each
    work-group's stream is at most 64 k-tiles (2 x K / 32), and run as two
    calls beyond; the results are the same bits either way."""
    os.environ.pop("ORMI_GEMM_PAIR", None)
    rng = np.random.default_rng(K)
    p0 = Problem(dev, rng, "dx", 1024, 4096, K, MUL_FN_D)
    p1 = Problem(dev, rng, "dw", 4096, 1024, K, ADD)
    g, got, want = pair_vs_each(dev, p0, p1)
    assert g == grouped
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)


def test_calls_that_do_not_group_run_in_order(dev):
    rng = np.random.default_rng(8)
    big = (1024, 4096, 256)
    cases = {
        # fewer tiles than compute units: the product alone takes other tiles
        "small": (Problem(dev, rng, "dx", 512, 1024, 256), Problem(dev, rng, "dw", *big)),
        "activation": (Problem(dev, rng, "dx", *big, UNARY), Problem(dev, rng, "dw", *big)),
        "layouts": (Problem(dev, rng, "nn", *big), Problem(dev, rng, "nn", *big)),
    }
    for name, (p0, p1) in cases.items():
        g, got, want = pair_vs_each(dev, p0, p1)
        assert g == 0, name
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b, err_msg=name)
    os.environ["ORMI_GEMM_PAIR"] = "0"
    try:
        p0, p1 = Problem(dev, rng, "dx", *big), Problem(dev, rng, "dw", *big)
        g, got, want = pair_vs_each(dev, p0, p1)
        assert g == 0
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b)
    finally:
        os.environ.pop("ORMI_GEMM_PAIR", None)


def test_dependent_products_run_in_order(dev):
    """Product 1 reads product 0's output as its A: not independent, so the
    pair runs as two calls and product 1 sees product 0's result."""
    rng = np.random.default_rng(9)
    M, N, K = 2048, 2048, 2048
    p0 = Problem(dev, rng, "dx", M, N, K)
    p1 = Problem(dev, rng, "dw", M, N, K)
    p1.desc.a, p1.desc.a_stride_m, p1.desc.a_stride_k = p0.desc.c, 1, M  # A1 = C0^T (a view of C0)
    g = run_pair(dev, p0, p1)
    assert g == 0
    c1 = p1.result()
    p1.reset()
    run_each(dev, p1)  # reads C0 as product 0 left it
    np.testing.assert_array_equal(p1.result(), c1)
    check_rows(p0, p0.result())
    # and product 1 overwriting an operand product 0 reads: also in order
    q0 = Problem(dev, rng, "dx", M, N, K)
    q1 = Problem(dev, rng, "dw", M, N, K)
    q1.desc.c = q0.desc.a  # C1 is A0's buffer (both M x K = 2048 x 2048 floats)
    assert run_pair(dev, q0, q1) == 0


def test_invalid_descriptor_launches_nothing(dev):
    rng = np.random.default_rng(10)
    p0 = Problem(dev, rng, "dx", 1024, 4096, 256)
    p1 = Problem(dev, rng, "dw", 4096, 1024, 256)
    p1.desc.M = -1
    grouped = ctypes.c_int(-1)
    rc = dev.lib.ormi_hip_gemm_pair(ctypes.byref(p0.desc), ctypes.byref(p0.epi), ctypes.byref(p1.desc),
                                    ctypes.byref(p1.epi), ctypes.byref(grouped))
    assert rc != 0 and b"negative" in dev.lib.ormi_hip_last_error()
    assert grouped.value == 0
    np.testing.assert_array_equal(p0.result(), p0.c0)  # product 0 did not run either


# ------------------------------------------------------------- scheduler --
def c5_step(dev, seed=4, batch=1024, dims=(1024, 4096, 4096, 1024)):
    """The C5 training step with its updates and loss realized together (as
    the bench runs it); returns the new weights, the loss and the step's
    grouped launches."""
    import math

    from ormi_amd import Tensor, realize_all
    from ormi_amd import ormi_backend as ob

    rng = np.random.default_rng(seed)
    X = Tensor(rng.normal(0, 1, (batch, dims[0])).astype(np.float32), dev)
    Y = Tensor(rng.normal(0, 1, (batch, dims[-1])).astype(np.float32), dev)
    ws = [Tensor(rng.uniform(-math.sqrt(6 / i), math.sqrt(6 / i), (i, o)).astype(np.float32), dev, requires_grad=True)
          for i, o in zip(dims, dims[1:])]
    h = X
    for i, w in enumerate(ws):
        h = h @ w
        if i < len(ws) - 1:
            h = h.gelu()
    d = h - Y
    loss = (d * d).sum() * (1.0 / (batch * dims[-1]))
    loss.backward()
    ups = [w - w.grad * 1e-3 for w in ws]
    before = ob.gemm_pair_count()
    realize_all(*ups, loss)
    pairs = ob.gemm_pair_count() - before
    return [u.numpy() for u in ups], loss.numpy(), pairs


def with_pair_mode(mode, fn):
    saved = os.environ.get("ORMI_GEMM_PAIR")
    try:
        if mode is None:
            os.environ.pop("ORMI_GEMM_PAIR", None)
        else:
            os.environ["ORMI_GEMM_PAIR"] = mode
        return fn()
    finally:
        if saved is None:
            os.environ.pop("ORMI_GEMM_PAIR", None)
        else:
            os.environ["ORMI_GEMM_PAIR"] = saved


def test_scheduler_pairs_each_layers_backward_products(cabi, hip):
    """C5 at config size: the scheduler offers dZ2 = (dY W3^T) gelu'(Z2) with
    W3 - lr H2^T dY, and dZ1 with W2 - lr H1^T dZ2 (W1's update has no partner
    left). Grouped on request (ORMI_GEMM_PAIR=2) they are two launches per
    step; by default layer 3's pair (64 k-tiles per work-group) is grouped and
    layer 2's (256) runs as two calls. No bit of the step's results changes:
    weights and loss equal those with ORMI_GEMM_PAIR=0."""
    w2, l2, pairs2 = with_pair_mode("2", lambda: c5_step("hip"))
    assert pairs2 == 2, pairs2
    w1, l1, pairs1 = with_pair_mode(None, lambda: c5_step("hip"))
    assert pairs1 == 1, pairs1
    w0, l0, pairs0 = with_pair_mode("0", lambda: c5_step("hip"))
    assert pairs0 == 0
    for a, b, c in zip(w2, w1, w0):
        np.testing.assert_array_equal(a, c)
        np.testing.assert_array_equal(b, c)
    np.testing.assert_array_equal(l2, l0)
    np.testing.assert_array_equal(l1, l0)


def wide_layer_step(dev, seed=12, batch=512, n_in=8192, n_out=512):
    """One layer, Z = X W with X a trainable input: its backward's dX = dZ W^T
    (512 x 8192, K 512) and dW = X^T dZ (8192 x 512, K 512) are 256 tiles of
    16 k-tiles each, a pair shallow enough to group by default. X's gradient
    and W's SGD update are realized together with the loss."""
    import math

    from ormi_amd import Tensor, realize_all
    from ormi_amd import ormi_backend as ob

    rng = np.random.default_rng(seed)
    X = Tensor(rng.normal(0, 1, (batch, n_in)).astype(np.float32), dev, requires_grad=True)
    W = Tensor(rng.uniform(-math.sqrt(6 / n_in), math.sqrt(6 / n_in), (n_in, n_out)).astype(np.float32), dev,
               requires_grad=True)
    h = (X @ W).gelu()
    loss = (h * h).sum() * (1.0 / (batch * n_out))
    loss.backward()
    w_new = W - W.grad * 1e-3
    before = ob.gemm_pair_count()
    realize_all(w_new, X.grad, loss)
    return [w_new.numpy(), X.grad.numpy()], loss.numpy(), ob.gemm_pair_count() - before


def test_scheduler_groups_a_shallow_pair_by_default(cabi, hip):
    got, l1, pairs = with_pair_mode(None, lambda: wide_layer_step("hip"))
    assert pairs == 1, pairs
    want, l0, pairs0 = with_pair_mode("0", lambda: wide_layer_step("hip"))
    assert pairs0 == 0
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(l1, l0)


def test_empty_and_zero_depth_products_run_alone(dev):
    """A product with no elements launches nothing and its partner runs as its
    own call; a product of depth 0 (C = 0 through its epilogue) is not
    eligible, so the two run in order; a null descriptor is an error."""
    rng = np.random.default_rng(11)
    p1 = Problem(dev, rng, "dw", 4096, 1024, 256, ADD)
    empty = Problem(dev, rng, "dx", 128, 128, 64)
    empty.desc.M = 0
    p1.reset()
    assert run_pair(dev, empty, p1) == 0
    got = p1.result()
    p1.reset()
    run_each(dev, p1)
    np.testing.assert_array_equal(got, p1.result())

    z = Problem(dev, rng, "dx", 1024, 4096, 64, MUL_FN_D)
    z.desc.K = 0  # the product is 0: C = 0 * gelu'(D)
    z.reset(), p1.reset()
    assert run_pair(dev, z, p1) == 0
    np.testing.assert_array_equal(z.result(), np.zeros((1024, 4096), np.float32) * 0)
    grouped = ctypes.c_int(-1)
    rc = dev.lib.ormi_hip_gemm_pair(None, None, ctypes.byref(p1.desc), ctypes.byref(p1.epi), ctypes.byref(grouped))
    assert rc != 0 and b"null descriptor" in dev.lib.ormi_hip_last_error()


def random_net_step(dev, seed):
    """A random MLP step at widths where the backward products can pair
    (1024-4096 wide, batch 1024 or 2048): random activations, biases and loss,
    updates and loss realized together. Returns the new parameters, the loss
    and the step's grouped launches."""
    import math

    from ormi_amd import Tensor, realize_all
    from ormi_amd import ormi_backend as ob

    rng = np.random.default_rng(700 + seed)
    L = int(rng.integers(2, 4))
    dims = [int(rng.choice([1024, 2048, 4096])) for _ in range(L + 1)]
    n = int(rng.choice([1024, 2048]))
    acts = [str(rng.choice(["none", "relu", "tanh", "gelu"])) for _ in range(L)]
    X = Tensor(rng.standard_normal((n, dims[0])).astype(np.float32), dev)
    Y = Tensor(rng.standard_normal((n, dims[-1])).astype(np.float32), dev)
    Ws = [Tensor((rng.standard_normal((i, o)) / math.sqrt(i)).astype(np.float32), dev, requires_grad=True)
          for i, o in zip(dims, dims[1:])]
    bs = [Tensor(rng.standard_normal(o).astype(np.float32) * 0.1, dev, requires_grad=True) if rng.random() < 0.3 else None
          for o in dims[1:]]
    h = X
    for W, b, act in zip(Ws, bs, acts):
        h = h @ W
        if b is not None:
            h = h + b
        if act != "none":
            h = getattr(h, act)()
    if rng.random() < 0.5:
        d = h - Y
        loss = (d * d).sum() * (1.0 / (n * dims[-1]))
    else:
        loss = (h * Y).sum() * 0.5
    loss.backward()
    params = Ws + [b for b in bs if b is not None]
    ups = [p - p.grad * 1e-3 for p in params]
    order = [int(i) for i in rng.permutation(len(ups))]
    before = ob.gemm_pair_count()
    realize_all(*[ups[i] for i in order], loss)
    pairs = ob.gemm_pair_count() - before
    out = [u.numpy() for u in ups] + [loss.numpy()]
    loss.zero_grad_graph()
    return out, pairs


def test_random_networks_pair_bit_identically(cabi, hip):
    """Six random networks: with every eligible pair grouped (ORMI_GEMM_PAIR=2)
    the parameters and loss are the same bits as with none (0); pairs form."""
    total = 0
    for seed in range(6):
        got, pairs = with_pair_mode("2", lambda: random_net_step("hip", seed))
        want, none = with_pair_mode("0", lambda: random_net_step("hip", seed))
        assert none == 0
        total += pairs
        for a, b in zip(got, want):
            np.testing.assert_array_equal(np.atleast_1d(a).view(np.uint32), np.atleast_1d(b).view(np.uint32))
    assert total > 0


def test_bf16_products_run_as_two_calls(dev):
    """The pair kernel is fp32: two bf16 products (fp32 output) are not grouped
    and give exactly what two ormi_hip_gemm_ex calls give."""
    rng = np.random.default_rng(13)

    def bf16(x):
        b = np.ascontiguousarray(x, np.float32).view(np.uint32)
        return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even

    def put16(x):
        h = bf16(x)
        p = ctypes.c_void_p()
        assert dev.lib.ormi_hip_malloc(ctypes.byref(p), h.nbytes) == 0
        assert dev.lib.ormi_hip_memcpy_h2d(p, h.ctypes.data, h.nbytes) == 0
        dev.bufs.append(p)
        return p

    descs = []
    for M, N, K in ((2048, 2048, 256), (2048, 2048, 512)):
        d = GemmDesc(dtype=3, M=M, N=N, K=K, a=put16(rng.standard_normal((M, K))), a_stride_m=K, a_stride_k=1,
                     b=put16(rng.standard_normal((K, N))), b_stride_k=N, b_stride_n=1,
                     c=dev.put(np.zeros((M, N), np.float32)))
        descs.append(d)
    grouped = ctypes.c_int(-1)
    assert dev.lib.ormi_hip_gemm_pair(ctypes.byref(descs[0]), None, ctypes.byref(descs[1]), None,
                                      ctypes.byref(grouped)) == 0, dev.lib.ormi_hip_last_error()
    assert grouped.value == 0
    got = [dev.get(d.c, (d.M, d.N)) for d in descs]
    for d in descs:
        assert dev.lib.ormi_hip_gemm_ex(ctypes.byref(d), None) == 0
    for g, d in zip(got, descs):
        np.testing.assert_array_equal(g, dev.get(d.c, (d.M, d.N)))
