"""Element-wise consumers of a reduction stored by the reduction's own kernel.

mean is sum * (1/N), a scale applied as the sum is stored. The reference realizes the
SUM into a buffer and runs a second element-wise kernel over it
(csrc/backend/runtime.cpp:16-18, csrc/backend/cuda/kernels/reduce/sum.cu:
12-97). Here an element-wise region whose only non-scalar input is one SUM or
MAX of its own shape runs as that reduction's store epilogue. The kernel that
writes the reduced value (the finishing kernel of a split reduction) also
evaluates the region on it and writes the region's result. Both nodes then hold
buffers, and no kernel reads the reduction back.

The epilogue is lowered exactly as the element-wise kernel it replaces, so the
results are compared bit for bit with the unfused path (the reduction realized
first, then the element-wise kernel over its buffer), on row, column and global
reductions, one-pass and split. They are also checked against the CPU oracle.
The launch counter shows that the fused path launches only the reduction's
kernels. CPU: the generated kernels compile for gfx950."""
import zlib

import numpy as np
import pytest

from conftest import fp32_sum_tolerance


def T(data, dev, **kw):
    from ormi_amd import Tensor

    return Tensor(data, dev, **kw)


def bits(a):
    a = np.ascontiguousarray(a, np.float32)
    return a.view(np.uint32)


# shape, axis (None = all), keepdims: a row reduction (one pass), a column
# reduction (one pass), a few long rows (split, finishing kernel), a tall
# column reduction (split), a global reduction (split).
CASES = [((512, 1024), 1, False), ((256, 768), 0, True), ((8, 65536), 1, True), ((65536, 16), 0, False),
         ((1024, 1024), None, False)]


# ------------------------------------------------------------------- CPU --
@pytest.mark.parametrize("shape,axis,keepdims", CASES)
def test_mean_plans_one_reduction_with_a_store_epilogue(ob, cpu, cabi, shape, axis, keepdims):
    from test_cabi_codegen import _compile_only

    x = T(np.zeros(shape, np.float32), cpu)
    d = ob._plan_kernel(x.mean(axis, keepdims)._node)
    assert d.get("store_epilogue"), d["plan"]
    src = d["second_source"] if d["two_pass"] else d["source"]
    assert "epo[" in src
    for s in [d["source"]] + ([d["second_source"]] if d["two_pass"] else []):
        rc, _ = _compile_only(cabi, s, ob._rtc_options())
        assert rc == 0, cabi.ormi_hip_last_error()


def test_regions_that_are_not_store_epilogues(ob, cpu):
    """A non-scalar operand, a broadcast to a larger shape, two reductions, an
    argmax: the region stays an element-wise kernel of its own."""
    x = T(np.zeros((64, 32), np.float32), cpu)
    y = T(np.zeros((64,), np.float32), cpu)
    assert ob._is_store_epilogue((x.sum(1) * 0.5)._node)
    assert ob._is_store_epilogue(((x.max(0) - 1.0).exp())._node)
    for node in [(x.sum(1) * y)._node, (x - x.max(1, keepdims=True))._node,
                 (x.sum(1) + x.max(1))._node, (x.argmax(1).astype("float32") * 2.0)._node,
                 (x.sum(1) * 0.5).astype("int32")._node]:
        assert not ob._is_store_epilogue(node)


# ------------------------------------------------------------------- GPU --
def unfused(X, fn, red):
    s = red(X)
    s.realize()
    return s, fn(s)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,axis,keepdims", CASES)
def test_mean_is_one_kernel_and_matches_the_unfused_bits(ob, cpu, hip, shape, axis, keepdims):
    rng = np.random.default_rng(sum(shape) + (axis or 7))
    x = rng.normal(0, 2, shape).astype(np.float32)
    X = T(x, hip)
    n = x.size if axis is None else shape[axis]

    s_ref, m_ref = unfused(X, lambda s: s * (1.0 / n), lambda X: X.sum(axis, keepdims))
    want = m_ref.numpy()

    X.realize()
    s = X.sum(axis, keepdims)
    m = s * (1.0 / n)
    plan = ob._plan_kernel(m._node)
    assert plan.get("store_epilogue")
    before = ob._kernel_launches()
    got = m.numpy()
    launched = ob._kernel_launches() - before
    assert launched == (2 if plan["two_pass"] else 1), launched
    assert s._node.is_realized  # the sum's own result is stored too
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(s.numpy()), bits(s_ref.numpy()))
    # the Tensor API's mean is this node
    assert np.array_equal(bits(X.mean(axis, keepdims).numpy()), bits(want))
    # and the oracle, within the fp32 sum bound scaled by 1/n
    oracle_mean = T(x, cpu).mean(axis, keepdims).numpy()
    exact = x.astype(np.float64).sum(axis=axis, keepdims=keepdims) / n
    tol = fp32_sum_tolerance(x, axis).reshape(exact.shape) / n + np.abs(exact) * np.finfo(np.float32).eps
    assert np.all(np.abs(got - exact) <= tol)
    assert np.all(np.abs(oracle_mean - exact) <= tol)


EPILOGUES = {
    "affine": lambda s: (s - 1.5) * 0.25,
    "relu_scale": lambda s: (s * 0.5).relu(),
    "tanh": lambda s: s.tanh() * 2.0,
    "exp_neg": lambda s: (-s * 0.01).exp(),
    "div": lambda s: 3.0 / (s * s + 1.0),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(EPILOGUES))
@pytest.mark.parametrize("red", ["sum", "max"])
@pytest.mark.parametrize("shape,axis,keepdims", CASES[:4])
def test_epilogue_regions_match_the_unfused_bits(ob, hip, name, red, shape, axis, keepdims):
    fn = EPILOGUES[name]
    rng = np.random.default_rng(zlib.crc32(f"{name}{red}{shape}".encode()))
    X = T(rng.normal(0, 1, shape).astype(np.float32), hip)
    reduce = (lambda X: X.sum(axis, keepdims)) if red == "sum" else (lambda X: X.max(axis, keepdims))
    _, ref = unfused(X, fn, reduce)
    want = ref.numpy()
    out = fn(reduce(X))
    assert ob._plan_kernel(out._node).get("store_epilogue")
    assert np.array_equal(bits(out.numpy()), bits(want)), (name, red)


@pytest.mark.gpu
def test_epilogue_scalar_operands_of_other_dtypes(ob, hip):
    """A 0-d bf16 leaf and a 1-element fp16 leaf as epilogue operands: read and
    converted as the element-wise kernel reads them."""
    rng = np.random.default_rng(5)
    X = T(rng.normal(0, 1, (300, 500)).astype(np.float32), hip)
    a = T(np.float32(0.3), hip, dtype="bfloat16")
    b = T(np.array([1.7], np.float32), hip, dtype="float16")
    fn = lambda s: s * a + b  # noqa: E731
    _, ref = unfused(X, fn, lambda X: X.sum(1))
    out = fn(X.sum(1))
    assert ob._plan_kernel(out._node).get("store_epilogue")
    assert np.array_equal(bits(out.numpy()), bits(ref.numpy()))


@pytest.mark.gpu
def test_epilogue_with_a_fused_prologue(ob, cpu, hip):
    """A row mean of exp(x - max), C3's softmax denominator scaled: the
    producer runs as the reduction's prologue and the scale as its epilogue,
    with no kernel of their own."""
    rng = np.random.default_rng(6)
    x = rng.normal(0, 2, (1024, 2048)).astype(np.float32)
    X = T(x, hip)
    mx = X.max(1, keepdims=True).realize()
    out = (X - mx).exp().mean(1)
    plan = ob._plan_kernel(out._node)
    assert plan.get("store_epilogue")
    before = ob._kernel_launches()
    got = out.numpy()
    assert ob._kernel_launches() - before == (2 if plan["two_pass"] else 1)
    s = (X - mx).exp().sum(1).realize()
    assert np.array_equal(bits(got), bits((s * (1.0 / 2048)).numpy()))


@pytest.mark.gpu
def test_regions_that_are_not_epilogues_still_compute(ob, hip):
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (128, 96)).astype(np.float32)
    y = rng.normal(0, 1, (128,)).astype(np.float32)
    X, Y = T(x, hip), T(y, hip)
    assert not ob._is_store_epilogue((X.sum(1) * Y)._node)
    got = (X.sum(1) * Y).numpy()
    s = X.sum(1).numpy()
    assert np.array_equal(bits(got), bits(s * y))
    got2 = (X - X.max(1, keepdims=True)).numpy()
    assert np.array_equal(bits(got2), bits(x - x.max(1, keepdims=True)))
