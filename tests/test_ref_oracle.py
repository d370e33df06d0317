"""The restated CPU oracle against the reference's own CPU path.

oracle/_ref/libormi_ref.so is l-h-ha/Ormi's core and CPU backend compiled from
/root/reference by oracle/Makefile.ref (every source of the path as it lies,
the OpenBLAS sgemm excepted; oracle/ref_driver.cpp runs a program through the
reference's execute_graph and compute_gradients). These tests run the same
seeded programs through it and through the oracle ("cpu" device of this
repository's core, whose shape rules, adjoints and autograd are restated from
the reference) and require the same bits: every value and every gradient.
That checks the oracle's tape VM (csrc/backend/cpu/jit.cpp:12-85, lowerings
cpu/lowerings/pointwise.cpp:5-15), its sequential sum (cpu/kernels/reduce/
sum.cpp:8-64), the view rules and the reverse pass (csrc/core/autograd.cpp:
24-47, adjoints csrc/core/ops/**) against the reference's own code, not a
restatement of it.

The programs keep to the reference's op set (no relu/tanh/max/matmul: its CPU
sgemm needs OpenBLAS headers this image lacks) and to what its sum handles:
the reference reduces a buffer by its view's strides (sum.cpp:20-48), which
divides by zero on an expanded (stride-0) view and misreads a transposed one.
Autograd feeds such views to that sum whenever a broadcast ADD/SUB receives an
expanded or transposed gradient, so every broadcast ADD/SUB here is followed by
a unary op (whose adjoint yields a contiguous product) and every transpose or
sum block is entered through one. The library is built where the reference
sources are (this container) and travels prebuilt with the tree, so these tests
also run on the GPU box; they skip only when it was never built."""
import math

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.skipif(not oracle.ref_available(), reason="reference CPU path not built (oracle/_ref)")

UNARY = ["NEG", "SIN", "COS"]


def make_program(seed):
    rng = np.random.default_rng(seed)
    m, n = int(rng.choice([1, 3, 7, 16, 33])), int(rng.choice([2, 5, 8, 31, 64]))
    leaves = [
        (rng.uniform(-1, 1, (m, n)).astype(np.float32), True),    # 0 X
        (rng.uniform(-1, 1, (m, n)).astype(np.float32), True),    # 1 Y (the loss weight)
        (rng.uniform(-1, 1, (n,)).astype(np.float32), True),      # 2 row vector
        (rng.uniform(-1, 1, (m, 1)).astype(np.float32), True),    # 3 column vector
        (rng.uniform(0.5, 1.5, (m, n)).astype(np.float32), True),  # 4 positive (POW base, DIV denominator)
        (np.float32(rng.uniform(-1, 1)).reshape(()), False),       # 5 scalar
    ]
    ops = []

    def emit(op, a, b=-1, attr=(), keepdims=False):
        ops.append((op, a, b, list(attr), keepdims))
        return len(leaves) + len(ops) - 1

    def unary(h):
        r = rng.random()
        if r < 0.15:
            return emit("EXP", emit("SIN", h))           # bounded argument
        if r < 0.25:
            return emit("LOG", emit("EXP", emit("COS", h)))  # log of a positive value
        return emit(str(rng.choice(UNARY)), h)

    h = emit("SIN", 0)
    marks = [h]
    for _ in range(int(rng.integers(3, 9))):
        r = rng.random()
        if r < 0.25:
            h = unary(h)
        elif r < 0.6:
            op = str(rng.choice(["ADD", "SUB", "MUL", "DIV", "POW"]))
            if op == "POW":
                h = emit("POW", 4, h)                     # positive base
            elif op == "DIV":
                h = emit("DIV", h, 4)
            else:
                other = int(rng.choice([0, 2, 3, 5] + marks))
                h = emit(op, h, other) if rng.random() < 0.5 else emit(op, other, h)
            h = unary(h)                                   # contiguous gradient into the broadcast op
        elif r < 0.8 and m > 1 and n > 1:
            t = emit("TRANSPOSE", unary(h), attr=[1, 0])
            t = emit("TRANSPOSE", unary(t), attr=[1, 0])
            h = unary(t)
        else:
            # a row sum kept as (m, 1), or a column sum dropped to (n,): the
            # backward of a broadcast from (1, n) reads past a buffer in the
            # reference's sum (keepdims over axis 0, unbroadcast to a leading 1)
            axis = int(rng.integers(0, 2))
            s = emit("SUM", unary(h), attr=[axis], keepdims=axis == 1)
            h = emit("MUL", h, s)
        marks.append(h)
    loss = emit("SUM", emit("MUL", h, 1), attr=[0, 1], keepdims=False)
    return leaves, ops, marks, loss


def run_oracle(leaves, ops, outputs, grad_root):
    """The same program on the oracle ("cpu" device of this repository's core)."""
    from ormi_amd import Tensor, ormi_backend as ob

    nodes = [Tensor(a, "cpu", requires_grad=rg)._node for a, rg in leaves]
    for name, a, b, attr, keepdims in ops:
        if name == "SUM":
            nodes.append(ob.sum(nodes[a], attr, keepdims))
        elif name == "TRANSPOSE":
            nodes.append(ob.transpose(nodes[a], attr))
        elif name in ("ADD", "SUB", "MUL", "DIV", "POW"):
            nodes.append(getattr(ob, name.lower())(nodes[a], nodes[b]))
        else:
            nodes.append(getattr(ob, name.lower())(nodes[a]))
    if grad_root >= 0:
        ob.compute_gradients(nodes[grad_root])
    dev = Tensor(np.zeros(1, np.float32), "cpu").device
    res = []
    for o in outputs:
        node = nodes[o] if o >= 0 else nodes[-1 - o].grad
        res.append(None if node is None else np.asarray(Tensor._wrap(node, dev).numpy(), dtype=np.float32))
    return res


def same(a, b):
    """Bit-identical, NaN positions included (their payloads are not compared)."""
    if a is None or b is None:
        return a is None and b is None
    if a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.fixture(scope="module")
def cpu_oracle():
    oracle.load()
    return "cpu"


def test_reference_known_answers(cpu_oracle):
    """The driver itself on the reference's own KATs: (2+3)*4 = 20
    (csrc/tests/backend/cpu/test_jit.cpp:42-57), broadcast [2,3]+[3] -> 7
    (:59-73), axis-1 sum [6,15] (kernels/reduce/test_sum.cpp:30-89), and the
    gradients of sum(a*b) (ormi-core/tests/test_tensor.py:70-81)."""
    two, three, four = (np.full((2, 2), v, np.float32) for v in (2, 3, 4))
    r = oracle.ref_run([(two, False), (three, False), (four, False)], [("ADD", 0, 1, [], 0), ("MUL", 3, 2, [], 0)], [4])
    assert np.all(r[0] == 20)
    a = np.ones((2, 3), np.float32) * 3
    b = np.ones((3,), np.float32) * 4
    assert np.all(oracle.ref_run([(a, False), (b, False)], [("ADD", 0, 1, [], 0)], [2])[0] == 7)
    x = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    assert np.array_equal(oracle.ref_run([(x, False)], [("SUM", 0, -1, [1], 0)], [1])[0], [6, 15])
    p = np.array([2, 3], np.float32)
    q = np.array([5, 6], np.float32)
    ga, gb = oracle.ref_run([(p, True), (q, True)], [("MUL", 0, 1, [], 0), ("SUM", 2, -1, [0], 0)], [-1, -2],
                            grad_root=3)
    assert np.array_equal(ga, q) and np.array_equal(gb, p)


@pytest.mark.parametrize("seed", range(60))
def test_oracle_matches_the_reference_bit_for_bit(cpu_oracle, seed):
    leaves, ops, marks, loss = make_program(seed)
    grads = [-1 - i for i, (_, rg) in enumerate(leaves) if rg]
    outputs = marks + [loss] + grads
    want = oracle.ref_run(leaves, ops, outputs, grad_root=loss)
    got = run_oracle(leaves, ops, outputs, grad_root=loss)
    for k, (w, g) in enumerate(zip(want, got)):
        assert same(g, w), (seed, k, outputs[k])


def test_sum_orders_and_keepdims_match(cpu_oracle):
    """Reductions over every axis set of a 3-d contiguous input, with and
    without keepdims, at sizes where the sequential order shows in the bits."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((9, 130, 17)).astype(np.float32)
    cases = [([0], 0), ([1], 1), ([2], 0), ([0, 2], 1), ([0, 1, 2], 0), ([1, 2], 0)]
    ops = [("SUM", 0, -1, ax, kd) for ax, kd in cases]
    want = oracle.ref_run([(x, False)], ops, list(range(1, 1 + len(ops))))
    got = run_oracle([(x, False)], ops, list(range(1, 1 + len(ops))), -1)
    for (ax, kd), w, g in zip(cases, want, got):
        assert same(g, w), (ax, kd)
        assert math.isfinite(float(np.max(np.abs(w))))
    # the bits depend on the order: numpy's fp32 sum along a contiguous row
    # (eight interleaved partial sums, then pairwise) differs from the
    # reference's sequential one, which the oracle matches
    y = rng.standard_normal((64, 1000)).astype(np.float32)
    w1 = oracle.ref_run([(y, False)], [("SUM", 0, -1, [1], 0)], [1])[0]
    g1 = run_oracle([(y, False)], [("SUM", 0, -1, [1], 0)], [1], -1)[0]
    assert same(g1, w1) and not same(np.sum(y, axis=1, dtype=np.float32), w1)
