"""A broadcast of an unrealized one-element element-wise value is evaluated
inside the consuming kernel instead of being realized first.

The backward of a scaled sum (a loss: sum(...) * c, reference autograd
csrc/core/autograd.cpp:24-47 with the SUM adjoint's broadcast of the incoming
gradient) multiplies the one-element seed by c and broadcasts the product to
the summed input's shape through a view. The view is not element-wise, so it
used to be a region frontier: a kernel of ONE element ran first, then the
gradient's kernel read its buffer. Seen through, the view is the scalar, whose
region reads only one-element operands (read with stride 0 at any kernel
shape), so the gradient's kernel computes it itself: one launch instead of
two, and the same bits, since the same fp32 operations round the same way.

CPU: the gradient's region now plans as one kernel (before, planning it threw:
its input was not realized); a view of a large region, of a one-element
reduction, or of a one-element region longer than 16 ops stays a frontier.
GPU: launch counts, and bit-exact results against the unfused path (the
scalar realized first) and the oracle."""
import numpy as np
import pytest


def T(data, dev, **kw):
    from ormi_amd import Tensor

    return Tensor(data, dev, **kw)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def loss_grad(dev, x, c=0.25):
    X = T(x, dev, requires_grad=True)
    loss = (X * X).sum() * c
    loss.backward()
    return X, loss


# ------------------------------------------------------------------- CPU --
def test_backward_of_a_scaled_sum_plans_as_one_kernel(ob, cpu):
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    X, _ = loss_grad(cpu, x)
    d = ob._plan_kernel(X.grad._node)  # raised before: the scalar view was an unrealized input
    assert not d["two_pass"]


def test_explicit_broadcast_of_a_scalar_chain(ob, cpu):
    x = T(np.ones((64, 32), np.float32), cpu)
    s = (T(np.float32(3.0), cpu) * 0.5 + 1.0).reshape((1, 1)).expand((64, 32))
    d = ob._plan_kernel((x * s)._node)
    assert not d["two_pass"]


def _plan_raises(ob, node):
    try:
        ob._plan_kernel(node)
    except RuntimeError as e:
        assert "not realized" in str(e)
        return True
    return False


def test_views_of_non_scalars_and_reductions_stay_frontiers(ob, cpu):
    x = T(np.ones((8, 4), np.float32), cpu)
    big = (x * 2.0).transpose()  # a view of a 32-element region: realized first
    assert _plan_raises(ob, (big + 1.0)._node)
    red = x.sum().reshape((1, 1)).expand((8, 4))  # a one-element reduction: its own kernel
    assert _plan_raises(ob, (x * red)._node)
    long = T(np.float32(1.0), cpu)
    for _ in range(20):  # a one-element region of 20 ops: more than 16
        long = long * 1.0001
    assert _plan_raises(ob, (x * long.reshape((1, 1)).expand((8, 4)))._node)


# ------------------------------------------------------------------- GPU --
@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1024, 1024), (300, 7), (4096,)])
def test_scaled_sum_gradient_is_one_kernel_and_bit_exact(ob, cpu, hip, shape):
    rng = np.random.default_rng(sum(shape))
    x = rng.normal(0, 1, shape).astype(np.float32)
    X, _ = loss_grad(hip, x)
    before = ob._kernel_launches()
    g = X.grad.numpy()
    assert ob._kernel_launches() - before == 1
    # d((x x) sum c)/dx = c x + c x in fp32, c a power of two: exact
    c = np.float32(0.25)
    np.testing.assert_array_equal(bits(g), bits(c * x + c * x))
    Xc, _ = loss_grad(cpu, x)
    np.testing.assert_array_equal(bits(g), bits(Xc.grad.numpy()))


@pytest.mark.gpu
def test_scalar_chain_matches_the_realized_scalar(ob, hip):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (512, 256)).astype(np.float32)
    X = T(x, hip)
    a = T(np.float32(0.3), hip)

    def scalar():
        return ((a * 1.7 + 0.1).exp() / 3.0).tanh()

    fused = X * scalar().reshape((1, 1)).expand((512, 256))
    before = ob._kernel_launches()
    got = fused.numpy()
    assert ob._kernel_launches() - before == 1
    s = scalar().realize()  # the unfused path: the scalar's own kernel, then the product
    want = (X * s.reshape((1, 1)).expand((512, 256))).numpy()
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.gpu
def test_scalar_view_in_a_reduction_prologue_and_a_grouped_realize(ob, hip):
    """The scalar is also evaluated inside a reduction's prologue (one kernel for
    sum(x * s) over rows) and inside a multi-output kernel of realize_all."""
    from ormi_amd import realize_all

    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (256, 1024)).astype(np.float32)
    X = T(x, hip)
    a = T(np.float32(1.5), hip)

    def view():
        return (a * 0.5 - 0.25).reshape((1, 1)).expand((256, 1024))

    red = (X * view()).sum(1)
    plan = ob._plan_kernel(red._node)
    before = ob._kernel_launches()
    got = red.numpy()
    assert ob._kernel_launches() - before == (2 if plan["two_pass"] else 1)
    s = (a * 0.5 - 0.25).realize()
    want = (X * s.reshape((1, 1)).expand((256, 1024))).sum(1).numpy()
    np.testing.assert_array_equal(bits(got), bits(want))

    u, v = X * view(), X + view()
    before = ob._kernel_launches()
    realize_all(u, v)
    assert ob._kernel_launches() - before == 1
    np.testing.assert_array_equal(bits(u.numpy()), bits(x * np.float32(0.5)))
    np.testing.assert_array_equal(bits(v.numpy()), bits(x + np.float32(0.5)))
