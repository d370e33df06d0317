"""The HIP device behind the reference's own core.

oracle/_ref/libormi_ref_hip.so is l-h-ha/Ormi's core and CPU backend, compiled
from /root/reference by oracle/Makefile.ref with the maintainer's edits that
add a device (oracle/ref_hip_device.sh: DeviceEnum::HIP, the get_allocator
case of csrc/core/allocator.cpp:5-12, the execute_graph case of
csrc/backend/runtime.cpp:29-38), the HIP glue of ormi_amd/csrc/ormi_core_hip
(HIPAllocator, hip::execute_jit over ormi_hip_map, the MATMUL and SUM graph
breakers over ormi_hip_gemm and ormi_hip_reduce), and oracle/ref_driver.cpp.
It links against libormi_hip.so and nothing else of this repository, so these
tests run the reference's graph, autograd and runtime unchanged on the HIP
device: the drop-in claim itself.

The checks:
  - without a GPU the device is absent the way the reference's test fixture
    expects (get_allocator throws, csrc/tests/test_utils.h:17-21), and the CPU
    device of the edited core still gives the reference's own bits;
  - on the GPU (-m gpu): every known-answer vector of the reference's tests,
    exactly; element-wise programs of + - * / (broadcasts, scalars, transposed
    and reshaped views, their gradients) bit for bit against the reference's
    CPU device; each of exp/log/sin/cos/pow within rtol 1e-6; seeded programs
    with sums and gradients (tests/test_ref_oracle.py's generator) within the
    summation-order tolerance; GEMMs forward and backward, the C4 fp32 config
    included, within 2K eps32 |A||B| of a float64 product; a config-size
    row and column sum within the float64 sum's order bound; C1's shape and
    data in the reference's op set with its gradients; and a two-layer
    training step at C5's batch and widths (GEMMs, autograd, SGD update).
"""
import ctypes
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from test_ref_oracle import make_program, same

LIB = Path(oracle.__file__).resolve().parent / "_ref" / "libormi_ref_hip.so"
pytestmark = pytest.mark.skipif(not LIB.exists(), reason="reference core with the HIP device not built")

EPS32 = float(np.finfo(np.float32).eps)


@pytest.fixture(scope="module")
def refhip():
    return oracle.load_ref_library(LIB)


@pytest.fixture(scope="module")
def refcpu():
    return oracle.load_ref_library(oracle._REF_LIB)


def run(handle, device, leaves, ops, outputs, grad_root=-1, capacity=0):
    return oracle.ref_call(handle, device, leaves, ops, outputs, grad_root, capacity)


# ------------------------------------------------------------------ CPU tests --

def test_library_links_libormi_hip_only():
    """The edited reference core reaches this repository through the C ABI
    only: libormi_hip.so is its one dependency from here."""
    out = subprocess.run(["readelf", "-d", str(LIB)], capture_output=True, text=True, check=True).stdout
    needed = [l.split("[")[1].rstrip("]") for l in out.splitlines() if "(NEEDED)" in l]
    ours = [n for n in needed if "ormi" in n]
    assert ours == ["libormi_hip.so"], needed


def test_device_probe_follows_the_reference_fixture(refhip, cabi):
    """Without a GPU, get_allocator(DeviceEnum::HIP) throws (the HIPAllocator
    constructor's ormi_hip_init fails), so the reference's fixture would leave
    the device out; with one, the allocator is made. The CPU device is always
    there."""
    count = ctypes.c_int(-1)
    assert cabi.ormi_hip_device_count(ctypes.byref(count)) == 0
    ok, msg = oracle.ref_device_available(refhip, "hip")
    if count.value == 0:
        assert not ok
        assert msg.startswith("HIP Error") and "no GPU" in msg, msg
    else:
        assert ok, msg
    assert oracle.ref_device_available(refhip, "cpu") == (True, "")
    # the unedited reference has no HIP case at all
    ok, msg = oracle.ref_device_available(oracle.load_ref_library(oracle._REF_LIB), "hip")
    assert not ok and "Unsupported DeviceEnum" in msg


@pytest.mark.parametrize("seed", range(12))
def test_edited_core_keeps_the_cpu_device_bits(refhip, refcpu, seed):
    """The edits add a device and change nothing else: the CPU device of the
    edited core matches the unedited reference bit for bit."""
    leaves, ops, marks, loss = make_program(seed)
    outputs = marks + [loss] + [-1 - i for i, (_, rg) in enumerate(leaves) if rg]
    want = run(refcpu, "cpu", leaves, ops, outputs, loss)
    got = run(refhip, "cpu", leaves, ops, outputs, loss)
    for k, (w, g) in enumerate(zip(want, got)):
        assert same(g, w), (seed, k)


# ------------------------------------------------------------------ GPU tests --

def kat_program(case):
    """A tests/golden/reference_kats.json case as a driver program."""
    names = list(case["inputs"])
    leaves = []
    for nm in names:
        spec = case["inputs"][nm]
        vals = np.array(spec["values"], np.float32)
        rg = bool(spec.get("requires_grad", False))
        if "strides" in spec:
            leaves.append((vals, rg, (list(spec["shape"]), list(spec["strides"]))))
        else:
            leaves.append((vals.reshape(spec["shape"]), rg))
    shapes = {i: list(case["inputs"][nm]["shape"]) for i, nm in enumerate(names)}
    ops = []

    def build(expr):
        if isinstance(expr, str):
            return names.index(expr)
        op, *args = expr
        if op in ("add", "sub", "mul", "div", "pow", "matmul"):
            a, b = build(args[0]), build(args[1])
            ops.append((op.upper(), a, b, [], 0))
        elif op in ("neg", "exp", "sin", "cos", "log"):
            ops.append((op.upper(), build(args[0]), -1, [], 0))
        elif op == "sum":
            ops.append(("SUM", build(args[0]), -1, list(args[1]), int(bool(args[2]))))
        elif op == "reshape":
            ops.append(("RESHAPE", build(args[0]), -1, list(args[1]), 0))
        elif op == "transpose":
            a = build(args[0])
            nd = len(shapes.get(a, [0, 0]))
            ops.append(("TRANSPOSE", a, -1, list(reversed(range(nd))), 0))
        else:
            raise ValueError(op)
        return len(leaves) + len(ops) - 1

    root = build(case["expr"])
    return names, leaves, ops, root


@pytest.mark.gpu
def test_reference_kats_through_the_reference_core(refhip):
    """Every known-answer vector of the reference's own tests, realized by the
    reference's execute_graph / compute_gradients on DeviceEnum::HIP."""
    cases = json.loads((Path(__file__).resolve().parent / "golden" / "reference_kats.json").read_text())["cases"]
    ran = 0
    for case in cases:
        names, leaves, ops, root = kat_program(case)
        if "grads" in case:
            idx = {nm: i for i, nm in enumerate(names)}
            outs = [-1 - idx[nm] for nm in case["grads"]]
            got = run(refhip, "hip", leaves, ops, outs, grad_root=root)
            for nm, g in zip(case["grads"], got):
                assert g.reshape(-1).tolist() == [float(v) for v in case["grads"][nm]], (case["name"], nm, g)
        else:
            (got,) = run(refhip, "hip", leaves, ops, [root])
            exp = case["expect"]
            assert list(got.shape) == list(exp["shape"]), case["name"]
            want = np.array(exp["values"], np.float32)
            if case.get("atol") is None:
                assert got.reshape(-1).tolist() == want.tolist(), (case["name"], got)
            else:
                assert np.allclose(got.reshape(-1), want, atol=case["atol"], rtol=0), (case["name"], got)
        ran += 1
    assert ran == len(cases) > 20


def exact_program(seed):
    """+ - * / and NEG over full-shape leaves, a row vector, a column vector and
    a scalar, through transposed, reshaped and expanded views. Forward values
    are exact roundings of the same operations on either device. Gradients flow
    only into the full-shape leaves (the broadcast ones take none), so the
    backward is element-wise too (the loss SUM's adjoint is an expanded view)
    and exact as well."""
    rng = np.random.default_rng(500 + seed)
    m, n = int(rng.choice([2, 5, 16, 33])), int(rng.choice([3, 8, 31, 64]))
    leaves = [
        (rng.uniform(-1, 1, (m, n)).astype(np.float32), True),
        (rng.uniform(0.5, 1.5, (m, n)).astype(np.float32), True),
        (rng.uniform(-1, 1, (n,)).astype(np.float32), False),
        (rng.uniform(-1, 1, (m, 1)).astype(np.float32), False),
        (np.float32(rng.uniform(-2, 2)).reshape(()), False),
    ]
    ops = []

    def emit(op, a, b=-1, attr=()):
        ops.append((op, a, b, list(attr), 0))
        return len(leaves) + len(ops) - 1

    h = emit("MUL", 0, 1)
    marks = [h]
    for _ in range(int(rng.integers(4, 10))):
        r = rng.random()
        if r < 0.5:
            op = str(rng.choice(["ADD", "SUB", "MUL"]))
            other = int(rng.choice([0, 2, 3, 4] + marks))
            h = emit(op, h, other) if rng.random() < 0.5 else emit(op, other, h)
        elif r < 0.65:
            h = emit("DIV", h, 1)
        elif r < 0.75:
            h = emit("NEG", h)
        elif r < 0.9:
            t = emit("TRANSPOSE", h, attr=[1, 0])
            t = emit("MUL", t, emit("TRANSPOSE", 1, attr=[1, 0]))
            h = emit("TRANSPOSE", t, attr=[1, 0])
        else:
            t = emit("RESHAPE", emit("NEG", h), attr=[m * n])  # NEG: a contiguous value to reshape
            h = emit("RESHAPE", emit("ADD", t, emit("RESHAPE", 0, attr=[m * n])), attr=[m, n])
        marks.append(h)
    loss = emit("SUM", h, attr=[0, 1])
    return leaves, ops, marks, loss


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(20))
def test_exact_ops_are_bit_exact(refhip, refcpu, seed):
    leaves, ops, marks, loss = exact_program(seed)
    outputs = marks + [-1, -2]
    want = run(refcpu, "cpu", leaves, ops, outputs, loss)
    got = run(refhip, "hip", leaves, ops, outputs, loss)
    for k, (w, g) in enumerate(zip(want, got)):
        assert same(g, w), (seed, k, outputs[k])


@pytest.mark.gpu
@pytest.mark.parametrize("op", ["EXP", "LOG", "SIN", "COS", "POW"])
def test_transcendentals_within_rtol_1e6(refhip, refcpu, op):
    """Each op alone over 2^16 values, against the reference CPU device's host
    libm (csrc/backend/cpu/lowerings/pointwise.cpp:5-15)."""
    rng = np.random.default_rng(77)
    x = rng.uniform(-4, 4, (256, 256)).astype(np.float32)
    pos = rng.uniform(0.05, 4, (256, 256)).astype(np.float32)
    if op == "LOG":
        leaves, ops = [(pos, False)], [("LOG", 0, -1, [], 0)]
    elif op == "POW":
        leaves, ops = [(pos, False), (rng.uniform(-3, 3, (256, 256)).astype(np.float32), False)], [("POW", 0, 1, [], 0)]
    else:
        leaves, ops = [(x, False)], [(op, 0, -1, [], 0)]
    out = len(leaves)
    (want,) = run(refcpu, "cpu", leaves, ops, [out])
    (got,) = run(refhip, "hip", leaves, ops, [out])
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=0 if op in ("EXP", "POW") else 1e-7)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(30))
def test_seeded_programs_match_the_reference_cpu(refhip, refcpu, seed):
    """tests/test_ref_oracle.py's programs (transcendentals, broadcasts, views,
    row and column sums, the loss and every gradient) on DeviceEnum::HIP, next
    to the reference's CPU device, both against the program in float64. The two
    fp32 evaluations round differently (sequential against tree sums, host libm
    against the device's transcendentals), and a chain amplifies either by its
    own conditioning (a cosine of a sum of 16 exponentials, a product with a
    column sum), so no fixed rtol fits every output. The check is that the HIP
    device is as accurate as the reference's own CPU path: on every output its
    largest error against float64 is at most 4x the CPU path's, plus 2^-20 of
    the output's magnitude."""
    from numpy_autograd import run_program

    leaves, ops, marks, loss = make_program(seed)
    outputs = marks + [loss] + [-1 - i for i, (_, rg) in enumerate(leaves) if rg]
    want = run(refcpu, "cpu", leaves, ops, outputs, loss)
    got = run(refhip, "hip", leaves, ops, outputs, loss)
    exact = run_program(leaves, ops, outputs, loss)
    for k, (w, g, x) in enumerate(zip(want, got, exact)):
        assert (w is None) == (g is None) == (x is None), (seed, k)
        if w is None:
            continue
        assert g.shape == w.shape == x.shape, (seed, k)
        if not w.size:
            continue
        scale = float(np.max(np.abs(x)))
        err_cpu = float(np.max(np.abs(w - x)))
        err_hip = float(np.max(np.abs(g - x)))
        assert err_hip <= 4 * err_cpu + 2.0 ** -20 * scale, (seed, k, outputs[k], err_hip, err_cpu, scale)


def gemm_bound(a_abs, b_abs, k):
    return 2 * k * EPS32 * (a_abs @ b_abs)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(7, 5, 9), (64, 96, 80), (257, 130, 65), (2048, 1024, 4096)])
def test_matmul_forward_and_backward(refhip, shape):
    """Z = A @ B, loss = sum(Z * W): the reference's MATMUL breaker slot runs
    ormi_hip_gemm forward, and adjoint_matmul's dA = dZ Bt, dB = At dZ
    (csrc/core/ops/blas/matmul.cpp:86-124, dZ = W exactly) run it on
    transposed views. (2048, 1024, 4096) is the C4 fp32 config."""
    M, K, N = shape
    rng = np.random.default_rng(sum(shape))
    a = rng.normal(0, 1 / 64, (M, K)).astype(np.float32)
    b = rng.normal(0, 1 / 64, (K, N)).astype(np.float32)
    w = rng.normal(0, 1, (M, N)).astype(np.float32)
    leaves = [(a, True), (b, True), (w, False)]
    ops = [("MATMUL", 0, 1, [], 0), ("MUL", 3, 2, [], 0), ("SUM", 4, -1, [0, 1], 0)]
    z, da, db = run(refhip, "hip", leaves, ops, [3, -1, -2], grad_root=5, capacity=max(M * N, M * K, K * N))
    a64, b64, w64 = a.astype(np.float64), b.astype(np.float64), w.astype(np.float64)
    assert np.all(np.abs(z - a64 @ b64) <= gemm_bound(np.abs(a64), np.abs(b64), K))
    assert np.all(np.abs(da - w64 @ b64.T) <= gemm_bound(np.abs(w64), np.abs(b64.T), N))
    assert np.all(np.abs(db - a64.T @ w64) <= gemm_bound(np.abs(a64.T), np.abs(w64), M))


@pytest.mark.gpu
def test_matmul_views_and_batch_broadcast(refhip):
    """The trans rule and the batch rule of cuda::matmul (csrc/backend/cuda/
    kernels/blas/matmul.cu:47-68): an operand given as a transposed view, and a
    batched product whose B has a stride-0 batch dim (the reference's
    BatchedBroadcasting case with bigger extents), then a 3-d batch over a
    4-d one that broadcasts A."""
    rng = np.random.default_rng(3)
    a = rng.standard_normal((40, 24)).astype(np.float32)
    b = rng.standard_normal((40, 33)).astype(np.float32)
    # a^T @ b (A a transposed view) and b^T @ a (A a transposed view of the other)
    zt, zb = run(refhip, "hip", [(a, False), (b, False)],
                 [("TRANSPOSE", 0, -1, [1, 0], 0), ("TRANSPOSE", 1, -1, [1, 0], 0), ("MATMUL", 2, 1, [], 0),
                  ("MATMUL", 3, 0, [], 0)], [4, 5])
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    assert zt.shape == (24, 33) and zb.shape == (33, 24)
    assert np.all(np.abs(zt - a64.T @ b64) <= gemm_bound(np.abs(a64.T), np.abs(b64), 40))
    assert np.all(np.abs(zb - b64.T @ a64) <= gemm_bound(np.abs(b64.T), np.abs(a64), 40))
    # the same product with the transposed operand on the right: a^T (24,40) @ (b^T)^T
    (zr,) = run(refhip, "hip", [(a, False), (b, False)],
                [("TRANSPOSE", 0, -1, [1, 0], 0), ("TRANSPOSE", 1, -1, [1, 0], 0), ("TRANSPOSE", 3, -1, [1, 0], 0),
                 ("MATMUL", 2, 4, [], 0)], [5])
    assert np.array_equal(zr, zt)

    A = rng.standard_normal((3, 17, 12)).astype(np.float32)
    Bm = rng.standard_normal((12, 19)).astype(np.float32)
    # B as a (3, 12, 19) view with batch stride 0 over one (12, 19) buffer
    (z,) = run(refhip, "hip", [(A, False), (Bm, False, ([3, 12, 19], [0, 19, 1]))], [("MATMUL", 0, 1, [], 0)], [2])
    want = A.astype(np.float64) @ Bm.astype(np.float64)
    assert np.all(np.abs(z - want) <= gemm_bound(np.abs(A.astype(np.float64)), np.abs(Bm.astype(np.float64)), 12))

    A4 = rng.standard_normal((2, 1, 9, 8)).astype(np.float32)
    B3 = rng.standard_normal((3, 8, 5)).astype(np.float32)
    (z,) = run(refhip, "hip", [(A4, False), (B3, False)], [("MATMUL", 0, 1, [], 0)], [2])
    want = A4.astype(np.float64) @ B3.astype(np.float64)
    assert z.shape == (2, 3, 9, 5)
    assert np.all(np.abs(z - want) <= gemm_bound(np.abs(A4.astype(np.float64)), np.abs(B3.astype(np.float64)), 8))


@pytest.mark.gpu
def test_row_and_column_sums_at_config_width(refhip):
    """SUM over axis 1 and axis 0 of a (4096, 8192) N(0, 2) input (C3's row
    width), through the reference's SUM breaker slot: within the order bound
    n eps sum|x| of the float64 sum, the rtol 1e-5 contract of fp32 reductions."""
    rng = np.random.default_rng(2)
    x = rng.normal(0, 2, (4096, 8192)).astype(np.float32)
    rows, cols = run(refhip, "hip", [(x, False)], [("SUM", 0, -1, [1], 0), ("SUM", 0, -1, [0], 1)], [1, 2])
    x64 = x.astype(np.float64)
    ax = np.abs(x64)
    assert rows.shape == (4096,) and cols.shape == (1, 8192)
    assert np.all(np.abs(rows - x64.sum(1)) <= 8192 * EPS32 * ax.sum(1))
    assert np.all(np.abs(cols[0] - x64.sum(0)) <= 4096 * EPS32 * ax.sum(0))


@pytest.mark.gpu
def test_c1_shaped_program_through_the_reference_core(refhip, refcpu):
    """C1's shape and data (1024x1024, seed 0, U(-1,1)) in the reference's op set
    (it has no relu): y = sum((a*b + c) * 0.5, axis 1), loss = sum(y), and the
    gradients of loss w.r.t. a, b, c. The reference realizes each op as its own
    kernel here. The gradients are element-wise products of the seed (0.5 * b,
    0.5 * a, 0.5), bit-exact against the reference's CPU device; the row sums
    within n eps sum|v| of float64."""
    rng = np.random.default_rng(0)
    a, b, c = (rng.uniform(-1, 1, (1024, 1024)).astype(np.float32) for _ in range(3))
    half = np.float32(0.5).reshape(())
    leaves = [(a, True), (b, True), (c, True), (half, False)]
    ops = [("MUL", 0, 1, [], 0), ("ADD", 4, 2, [], 0), ("MUL", 5, 3, [], 0), ("SUM", 6, -1, [1], 0),
           ("SUM", 7, -1, [0], 0)]
    outputs = [7, 8, -1, -2, -3]
    want = run(refcpu, "cpu", leaves, ops, outputs, 8)
    got = run(refhip, "hip", leaves, ops, outputs, 8)
    for k in (2, 3, 4):
        assert same(got[k], want[k]), k
    v = ((a * b + c) * np.float32(0.5)).astype(np.float64)
    bound = 1024 * EPS32 * np.abs(v).sum(1)
    assert np.all(np.abs(got[0] - v.sum(1)) <= bound)
    assert abs(float(got[1].reshape(-1)[0]) - v.sum()) <= 1024 * 1024 * EPS32 * np.abs(v).sum()


@pytest.mark.gpu
def test_two_layer_training_step_through_the_reference_core(refhip):
    """C5's batch and widths without the activations the reference lacks:
    Y = (X W1) W2 with X (1024,1024), W1 (1024,4096), W2 (4096,1024), loss =
    sum((Y - T)^2) * 2^-20, the reference's autograd for dW1 and dW2 (two NT and
    two TN GEMMs over transposed views), then the SGD update W - lr dW, all on
    DeviceEnum::HIP. Checked against float64 normwise: the forward within
    2 K eps32 |A||B| per product, the updates and gradients within 1e-4."""
    rng = np.random.default_rng(4)
    X = rng.normal(0, 1, (1024, 1024)).astype(np.float32)
    T_ = rng.normal(0, 1, (1024, 1024)).astype(np.float32)
    W1 = rng.uniform(-np.sqrt(6 / 1024), np.sqrt(6 / 1024), (1024, 4096)).astype(np.float32)
    W2 = rng.uniform(-np.sqrt(6 / 4096), np.sqrt(6 / 4096), (4096, 1024)).astype(np.float32)
    scale = np.float32(2.0 ** -20).reshape(())
    lr = np.float32(1e-3).reshape(())
    leaves = [(X, False), (W1, True), (W2, True), (T_, False), (scale, False), (lr, False)]
    ops = [("MATMUL", 0, 1, [], 0),    # 6  H = X W1
           ("MATMUL", 6, 2, [], 0),    # 7  Y = H W2
           ("SUB", 7, 3, [], 0),       # 8  D = Y - T
           ("MUL", 8, 8, [], 0),       # 9  D*D
           ("SUM", 9, -1, [0, 1], 0),  # 10
           ("MUL", 10, 4, [], 0)]      # 11 loss
    outputs = [6, 7, 11, -2, -3]
    H, Y, loss, dW1, dW2 = run(refhip, "hip", leaves, ops, outputs, 11, capacity=4096 * 1024)
    x64, w1, w2, t64 = (v.astype(np.float64) for v in (X, W1, W2, T_))
    h64 = x64 @ w1
    assert np.all(np.abs(H - h64) <= 2 * 1024 * EPS32 * (np.abs(x64) @ np.abs(w1)))
    y64 = H.astype(np.float64) @ w2
    assert np.all(np.abs(Y - y64) <= 2 * 4096 * EPS32 * (np.abs(H.astype(np.float64)) @ np.abs(w2)))
    d64 = (x64 @ w1) @ w2 - t64
    np.testing.assert_allclose(float(loss.reshape(-1)[0]), (d64 * d64).sum() * 2.0 ** -20, rtol=1e-5)
    g = 2 * d64 * 2.0 ** -20
    dw2 = h64.T @ g
    dw1 = x64.T @ (g @ w2.T)

    def normwise(got, want):
        return np.linalg.norm(got - want) / np.linalg.norm(want)

    assert normwise(dW2, dw2) < 1e-4 and normwise(dW1, dw1) < 1e-4
    # the SGD update W - lr * dW as reference ops over the realized gradients
    upd_leaves = [(W1, False), (dW1, False), (W2, False), (dW2, False), (lr, False)]
    upd_ops = [("MUL", 1, 4, [], 0), ("SUB", 0, 5, [], 0), ("MUL", 3, 4, [], 0), ("SUB", 2, 7, [], 0)]
    nW1, nW2 = run(refhip, "hip", upd_leaves, upd_ops, [6, 8], capacity=4096 * 1024)
    assert same(nW1, W1 - dW1 * np.float32(1e-3)) and same(nW2, W2 - dW2 * np.float32(1e-3))
