"""The CPU oracle, pinned before it is trusted.

1. The reference's own known-answer tests, restated (values from the cited files).
2. Closed forms and independent computations (numpy, float64) that a plausible
   mistake in the oracle would fail: a dropped term, a wrong stride, a wrong
   tie rule, a transposed operand.
"""
import math

import numpy as np
import pytest

from conftest import empty_tensor_cases, fp32_sum_tolerance


def T(data, dev="cpu", **kw):
    from ormi_amd import Tensor

    return Tensor(data, device=dev, **kw)


def filled(ob, shape, value):
    buf = ob.numpy_to_buffer(np.full(shape, value, np.float32), ob.DeviceEnum.CPU)
    return ob.Node(buf, False, ob.Device(ob.DeviceEnum.CPU, 0))


def with_view(ob, values, shape, strides):
    buf = ob.numpy_to_buffer(np.array(values, np.float32), ob.DeviceEnum.CPU)
    n = ob.Node(buf, False, ob.Device(ob.DeviceEnum.CPU, 0))
    n.view = ob.TensorView(list(shape), list(strides))
    return n


def out(ob, node):
    return ob.buffer_to_numpy(node.data).reshape(-1)


# ---------------------------------------------------------------- reference KATs
def test_jit_kats(ob, cpu):
    """csrc/tests/backend/cpu/test_jit.cpp:26-99."""
    c = ob.add(filled(ob, [4], 2.0), filled(ob, [4], 3.0))
    ob.execute_jit(c)
    assert (out(ob, c) == 5.0).all()
    d = ob.mul(ob.add(filled(ob, [2, 2], 2.0), filled(ob, [2, 2], 3.0)), filled(ob, [2, 2], 4.0))
    ob.execute_jit(d)  # one tape of two ops
    assert (out(ob, d) == 20.0).all()
    e = ob.add(filled(ob, [2, 3], 2.0), filled(ob, [3], 5.0))
    ob.execute_jit(e)
    assert e.shape == [2, 3] and (out(ob, e) == 7.0).all()
    f = ob.add(filled(ob, [2, 2], 10.0), filled(ob, [], 3.0))
    ob.execute_jit(f)
    assert (out(ob, f) == 13.0).all()
    g = ob.sin(filled(ob, [2], 1.570796327))
    ob.execute_jit(g)
    assert np.allclose(out(ob, g), 1.0, atol=1e-5)


def test_sum_kats(ob, cpu):
    """csrc/tests/backend/cpu/kernels/reduce/test_sum.cpp:30-89."""
    x = T(np.arange(1, 7, dtype=np.float32).reshape(2, 3))
    assert x.sum().numpy() == 21.0
    assert x.sum(1).numpy().tolist() == [6.0, 15.0]
    assert x.sum(0, keepdims=True).numpy().tolist() == [[5.0, 7.0, 9.0]]
    cube = T(np.arange(1, 9, dtype=np.float32).reshape(2, 2, 2))
    assert cube.sum((0, 2)).numpy().tolist() == [14.0, 22.0]


def test_matmul_kats(ob, cpu):
    """csrc/tests/backend/cpu/kernels/blas/test_matmul.cpp:30-98."""
    a = with_view(ob, [1, 2, 3, 4, 5, 6], [2, 3], [3, 1])
    b = with_view(ob, [7, 8, 9, 10, 11, 12], [3, 2], [2, 1])
    c = ob.matmul(a, b)
    ob.execute_graph(c)
    assert out(ob, c).tolist() == [58, 64, 139, 154]
    a = with_view(ob, [1, 2, 3, 4, 5, 6], [3, 2], [1, 3])
    b = with_view(ob, [1, 2, 3, 4], [2, 2], [2, 1])
    c = ob.matmul(a, b)
    ob.execute_graph(c)
    assert out(ob, c).tolist() == [13, 18, 17, 24, 21, 30]
    a = with_view(ob, list(range(1, 13)), [2, 2, 3], [6, 3, 1])
    b = with_view(ob, [1, 2, 3, 4, 5, 6], [2, 3, 2], [0, 2, 1])
    c = ob.matmul(a, b)
    ob.execute_graph(c)
    assert out(ob, c).tolist() == [22, 28, 49, 64, 76, 100, 103, 136]


def test_graph_level_kats(ob, cpu):
    """csrc/tests/core/test_ops.cpp:25-160 and test_runtime.cpp:26-92."""
    c = ob.matmul(filled(ob, [2, 3], 2.0), filled(ob, [3, 2], 3.0))
    ob.execute_graph(c)
    assert (out(ob, c) == 18.0).all()
    a, b, cc = filled(ob, [2, 2], 2.0), filled(ob, [2, 2], 3.0), filled(ob, [2, 2], 4.0)
    ab = ob.add(a, b)
    d = ob.mul(ab, cc)
    ob.execute_graph(d)
    # The reference order realizes every intermediate (test_runtime.cpp:42).
    assert ab.is_realized and (out(ob, d) == 20.0).all()
    x = filled(ob, [2, 3, 4], 1.0)
    v = ob.reshape(x, [6, 4])
    ob.execute_graph(v)
    assert v.is_realized and v.data.ptr == x.data.ptr  # zero-copy view
    s = ob.sum(filled(ob, [2, 3], 2.0), [], False)
    ob.execute_graph(s)
    assert out(ob, s).tolist() == [12.0]


def test_python_api_kats(cpu):
    """ormi-core/tests/test_tensor.py:13-81 and example/test_matmul.py:19-25."""
    a, b = T([4.0, 6.0]), T([2.0, 3.0])
    assert (a + b).numpy().tolist() == [6, 9]
    assert (a - b).numpy().tolist() == [2, 3]
    assert (a * b).numpy().tolist() == [8, 18]
    assert (a / b).numpy().tolist() == [2, 2]
    assert (-a).numpy().tolist() == [-4, -6]
    assert (a ** 2.0).numpy().tolist() == [16, 36]
    a = T([2.0, 4.0])
    assert (10.0 + a).numpy().tolist() == [12, 14]
    assert (10.0 - a).numpy().tolist() == [8, 6]
    assert (10.0 * a).numpy().tolist() == [20, 40]
    assert (10.0 / a).numpy().tolist() == [5, 2.5]
    m = T([[1.0, 2.0], [3.0, 4.0]]) @ T([[2.0, 0.0], [0.0, 2.0]])
    assert m.numpy().tolist() == [[2, 4], [6, 8]]
    with pytest.raises(TypeError):
        _ = T([[1.0, 2.0]]) @ 2.0
    x = T([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
    assert x.reshape((3, 2)).numpy().tolist() == [[1, 2], [3, 4], [5, 6]]
    assert x.transpose().numpy().tolist() == [[1, 4], [2, 5], [3, 6]]
    a, b = T([2.0, 3.0], requires_grad=True), T([4.0, 5.0], requires_grad=True)
    ((a * b) + a).backward()
    assert a.grad.numpy().tolist() == [5, 6] and b.grad.numpy().tolist() == [2, 3]
    e = T([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]) @ T([[1.0], [2.0]])
    assert e.numpy().tolist() == [[5], [11], [17]]
    a = T([1.0], requires_grad=True)
    (a * 2.0).backward()
    assert a.grad is not None
    a.zero_grad()
    assert a.grad is None


# ------------------------------------------------- independent pins of the oracle
def test_pointwise_arithmetic_is_ieee_fp32(cpu):
    """+ - * / with no contraction equal numpy's float32 ops bit for bit."""
    rng = np.random.default_rng(10)
    a = rng.standard_normal((257,)).astype(np.float32)
    b = rng.standard_normal((257,)).astype(np.float32)
    c = rng.standard_normal((257,)).astype(np.float32)
    got = ((T(a) * T(b) + T(c)) / T(b) - T(a)).numpy()
    with np.errstate(all="ignore"):
        want = ((a * b + c) / b - a).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name,fn", [
    ("exp", np.exp), ("log", np.log), ("sin", np.sin), ("cos", np.cos), ("tanh", np.tanh),
    ("sigmoid", lambda x: 1 / (1 + np.exp(-x))),
    ("gelu", lambda x: 0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2)))),
    ("relu", lambda x: np.maximum(x, 0)),
])
def test_unary_against_float64(cpu, name, fn):
    rng = np.random.default_rng(11)
    x = rng.uniform(0.1 if name == "log" else -4, 4, 1000).astype(np.float32)
    got = getattr(T(x), name)().numpy().astype(np.float64)
    want = fn(x.astype(np.float64))
    assert np.allclose(got, want, rtol=4e-7, atol=1e-7), np.abs(got - want).max()


def test_activation_grads_against_finite_differences(cpu):
    rng = np.random.default_rng(12)
    x = rng.uniform(-3, 3, 64).astype(np.float64)
    h = 1e-3
    fns = {
        "tanh": np.tanh,
        "sigmoid": lambda v: 1 / (1 + np.exp(-v)),
        "gelu": lambda v: 0.5 * v * (1 + np.vectorize(math.erf)(v / math.sqrt(2))),
    }
    for name, f in fns.items():
        t = T(x.astype(np.float32), requires_grad=True)
        getattr(t, name)().sum().backward()
        fd = (f(x + h) - f(x - h)) / (2 * h)
        assert np.allclose(t.grad.numpy(), fd, atol=2e-4), name
    t = T(np.array([-1.0, 0.0, 2.0], np.float32), requires_grad=True)
    t.relu().sum().backward()
    assert t.grad.numpy().tolist() == [0.0, 0.0, 1.0]


def test_sum_against_float64(cpu):
    rng = np.random.default_rng(13)
    x = rng.normal(0, 2, (37, 129)).astype(np.float32)
    for axis in (None, 0, 1):
        got = T(x).sum(axis).numpy()
        want = x.astype(np.float64).sum(axis=axis)
        assert np.all(np.abs(got - want) <= fp32_sum_tolerance(x, axis))
    # Sequential fp32 order: the oracle equals an explicit left-to-right loop.
    row = x[3]
    acc = np.float32(0)
    for v in row:
        acc = np.float32(acc + v)
    assert T(x).sum(1).numpy()[3] == acc


def test_max_argmax_against_numpy(cpu):
    rng = np.random.default_rng(14)
    x = rng.integers(-5, 5, (23, 17)).astype(np.float32)  # many ties
    for axis in (0, 1):
        assert np.array_equal(T(x).argmax(axis).numpy(), np.argmax(x, axis=axis))
        assert np.array_equal(T(x).max(axis).numpy(), np.max(x, axis=axis))
    assert T(x).argmax().numpy() == np.argmax(x)
    y = x.copy()
    y[2, 5] = np.nan
    y[2, 9] = np.nan
    assert T(y).argmax(1).numpy()[2] == 5  # first NaN, as numpy
    assert np.isnan(T(y).max(1).numpy()[2])


def test_matmul_against_float64(cpu):
    rng = np.random.default_rng(15)
    a = rng.standard_normal((33, 70)).astype(np.float32)
    b = rng.standard_normal((70, 41)).astype(np.float32)
    got = (T(a) @ T(b)).numpy()
    want = a.astype(np.float64) @ b.astype(np.float64)
    bound = 70 * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b))
    assert np.all(np.abs(got - want) <= bound)
    # Transposed operands through views give the same numbers as numpy on the transposes.
    got_t = (T(a.T.copy()).transpose() @ T(b.T.copy()).transpose()).numpy()
    assert np.all(np.abs(got_t - want) <= bound)


def test_bf16_leaf_rounding(cpu):
    """Leaves created as bfloat16 hold round-to-nearest-even values."""
    vals = np.array([1.0, 1.00390625, 1.01171875, -3.14159, 1e-40, 65504.0], np.float32)
    got = T(vals, dtype="bfloat16").numpy()
    u = vals.view(np.uint32).astype(np.uint64)
    rne = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    assert np.array_equal(got.view(np.uint32), rne.astype(np.uint32))


def test_mlp_grads_against_float64(cpu):
    """Two-layer GELU MLP with MSE: oracle gradients equal a float64 hand derivation."""
    rng = np.random.default_rng(16)
    X = rng.standard_normal((8, 6)).astype(np.float32)
    W1 = rng.uniform(-0.5, 0.5, (6, 5)).astype(np.float32)
    W2 = rng.uniform(-0.5, 0.5, (5, 3)).astype(np.float32)
    Y = rng.standard_normal((8, 3)).astype(np.float32)
    w1, w2 = T(W1, requires_grad=True), T(W2, requires_grad=True)
    h = (T(X) @ w1).gelu()
    d = h @ w2 - T(Y)
    loss = (d * d).sum() * (1.0 / d.shape[0])
    loss.backward()
    erf = np.vectorize(math.erf)
    X64, W164, W264, Y64 = (v.astype(np.float64) for v in (X, W1, W2, Y))
    z = X64 @ W164
    hh = 0.5 * z * (1 + erf(z / math.sqrt(2)))
    dd = hh @ W264 - Y64
    g_out = 2 * dd / 8
    gW2 = hh.T @ g_out
    dh = g_out @ W264.T
    gelu_p = 0.5 * (1 + erf(z / math.sqrt(2))) + z * np.exp(-z * z / 2) / math.sqrt(2 * math.pi)
    gW1 = X64.T @ (dh * gelu_p)
    assert np.allclose(w2.grad.numpy(), gW2, rtol=1e-4, atol=1e-5)
    assert np.allclose(w1.grad.numpy(), gW1, rtol=1e-4, atol=1e-5)


# ------------------------------------------------- golden vectors (data fixtures)
def _kat_ids():
    from kat_runner import cases

    return [c["name"] for c in cases()]


@pytest.mark.parametrize("name", _kat_ids())
def test_golden_kats_on_oracle(ob, cpu, name):
    """tests/golden/reference_kats.json: the reference's own known answers."""
    from kat_runner import cases, run_case

    case = next(c for c in cases() if c["name"] == name)
    run_case(ob, case, ob.DeviceEnum.CPU)


def test_empty_tensors_follow_numpy(cpu):
    """0-length dims through maps, reductions, products and backward on the
    oracle, against numpy's results for the same operations."""
    import warnings

    got = empty_tensor_cases("cpu")
    z = lambda *s: np.zeros(s, np.float32)  # noqa: E731
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", RuntimeWarning)  # numpy's mean of nothing
        want = {
            "bcast_rows": z(0, 5) + np.ones(5, np.float32), "bcast_cols": z(3, 0) * 2, "bcast_both": z(0, 1) - np.ones((1, 7)),
            "unary": z(4, 0), "sum_rows": z(0, 5).sum(0), "sum_cols": z(0, 5).sum(1), "sum_all": z(0, 5).sum(),
            "sum_keep": z(2, 0, 3).sum(1, keepdims=True), "mean_empty": z(0, 5).mean(0), "max_kept_empty": z(0, 5).max(1),
            "matmul_k0": z(3, 0) @ z(0, 4), "matmul_m0": z(0, 3) @ np.ones((3, 4)), "matmul_n0": np.ones((3, 4)) @ z(4, 0),
            "matmul_batched_k0": z(2, 3, 0) @ z(2, 0, 5), "grad_a": z(0, 5), "grad_b": z(5), "grad_w": z(5, 3),
        }
    for name in ("max_over_empty", "argmax_over_empty"):
        assert got[name][0] == "error" and "zero-size" in got[name][1], (name, got[name])
    for name, w in want.items():
        g = got[name]
        assert not isinstance(g, tuple), (name, g)
        assert g.shape == np.shape(w), (name, g.shape, np.shape(w))
        np.testing.assert_array_equal(g, np.asarray(w, np.float32), err_msg=name)


def test_python_scalar_operands_share_leaves_but_keep_signed_zero(cpu):
    """Python scalars become cached 0-d leaves per (device, value) (a host-to-device
    copy saved per literal); -0.0 and 0.0 compare equal as floats but must stay
    distinct leaves."""
    from ormi_amd import Tensor

    x = Tensor(np.array([1.0, -2.0], np.float32), "cpu")
    assert (x * 0.5)._node.parents[1] is (x * 0.5)._node.parents[1]
    assert list(np.signbit((x * 0.0).numpy())) == [False, True]
    assert list(np.signbit((x * -0.0).numpy())) == [True, False]
    a, b = Tensor(np.ones(2, np.float32), "cpu"), Tensor(np.ones(2, np.float32), "cpu")
    assert (a + b).numpy().tolist() == [2.0, 2.0]  # tensors with separate Device objects
