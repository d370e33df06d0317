"""Gradients of seeded random graphs against an autograd that shares nothing
with the graph core (tests/numpy_autograd.py, float64, derivatives restated
from the mathematics).

The CPU oracle and the HIP device both run libormi_core.so's adjoints
(reference csrc/core/ops/**, csrc/core/adjoint.cpp:5-34, reverse pass
csrc/core/autograd.cpp:24-47), so checking one against the other cannot find a
wrong adjoint rule; this can. The graphs cover every differentiable op of the
core: + - x / and negation with broadcasting, exp, sin, cos, tanh, sigmoid,
gelu, scalar scaling, matmul (transposed and batch-broadcast operands), sum and
max over axes with and without keepdims, transpose, reshape, expand, relu.
Masks must not depend on rounding, so max acts on small-integer leaves (exact
ties) and relu on leaves kept at least 0.25 from zero; every other op is
smooth, denominators are at least 1 in magnitude, and magnitudes stay small
(operands in [-0.5, 0.5], scalings within 1.2, exp of a tanh), so no step is
ill-conditioned (sin of e^10 would amplify fp32 rounding to 1e-3). Each leaf's gradient must
match float64 within a normwise 1e-4 (fp32 rounding through at most a dozen
ops), and every element within 1e-3 of the gradient's largest magnitude.
"""
import numpy as np
import pytest

from numpy_autograd import V

UNARY = ["neg", "exp", "sin", "cos", "tanh", "sigmoid", "gelu"]


def make_case(seed):
    rng = np.random.default_rng(seed)
    m, k, n = (int(rng.choice([3, 8, 17, 32])) for _ in range(3))
    spec = {"seed": seed}
    leaves = {
        "X": rng.uniform(-0.5, 0.5, (m, k)).astype(np.float32),
        "W": rng.uniform(-0.5, 0.5, (k, n)).astype(np.float32),
        "b": rng.uniform(-1, 1, (n,)).astype(np.float32),
        "s": rng.uniform(0.5, 1.5, (m, 1)).astype(np.float32),
        "I": rng.integers(-3, 4, (m, n)).astype(np.float32),                       # max: exact ties
        "R": (rng.uniform(0.25, 1.0, (m, n)) * rng.choice([-1, 1], (m, n))).astype(np.float32),  # relu: no boundary
    }
    ops = []
    # a random smooth chain over the (m, n) product
    first = [("mm", ["X", "W"]), ("mmT", ["X", "W"])][int(rng.integers(0, 2))]
    ops.append(("h0",) + first)
    cur = "h0"
    for j in range(int(rng.integers(3, 8))):
        r = rng.random()
        out = f"h{j + 1}"
        if r < 0.3:
            ops.append((out, str(rng.choice(UNARY)), [cur]))
        elif r < 0.45:
            ops.append((out, "add", [cur, str(rng.choice(["b", "s"]))]))
        elif r < 0.6:
            ops.append((out, "mul", [cur, str(rng.choice(["b", "s", "I", "R"]))]))
        elif r < 0.7:
            ops.append((out, "sub", [cur, "b"]))
        elif r < 0.8:
            ops.append((out, "div", [cur, "den"]))
        elif r < 0.9:
            ops.append((out, "scale", [cur, float(rng.uniform(-1.2, 1.2))]))
        else:
            ops.append((out, "tr2", [cur]))  # transpose, tanh, transpose back
        cur = out
    # join with the masked terms
    axis, keep = int(rng.integers(0, 2)), bool(rng.random() < 0.5)
    ops.append(("mx", "max", ["I", axis, keep]))
    ops.append(("rl", "relu", ["R"]))
    ops.append(("j1", "mul", [cur, "rl"]))
    ops.append(("j2", "addmax", ["j1", "mx", axis, keep]))
    red = int(rng.integers(0, 3))
    ops.append(("out", "reduce", ["j2", red]))
    spec["ops"] = ops
    spec["leaves"] = leaves
    spec["w"] = rng.uniform(-1, 1, {0: (n,), 1: (m,), 2: (m, n)}[red]).astype(np.float32)
    return spec


def run(spec, mk, is_numpy):
    """Build the graph with tensors made by mk(name, array); return the loss node
    and the leaf tensors."""
    L = {name: mk(name, arr) for name, arr in spec["leaves"].items()}
    vals = dict(L)
    for out, op, args in spec["ops"]:
        a = vals[args[0]]
        if op == "mm":
            vals[out] = a @ vals[args[1]]
        elif op == "mmT":
            # the transposed-operand GEMMs autograd issues: (X^T)^T @ (W^T)^T
            vals[out] = a.transpose().transpose() @ vals[args[1]].transpose().transpose()
        elif op == "exp":
            vals[out] = a.tanh().exp()  # a bounded argument keeps the chain well conditioned
        elif op in UNARY:
            vals[out] = (-a) if op == "neg" else getattr(a, op)()
        elif op == "add":
            vals[out] = a + vals[args[1]]
        elif op == "sub":
            vals[out] = a - vals[args[1]]
        elif op == "mul":
            vals[out] = a * vals[args[1]]
        elif op == "div":
            vals[out] = a / (L["s"] * L["s"] + 1.0)
        elif op == "scale":
            vals[out] = a * args[1]
        elif op == "tr2":
            vals[out] = a.transpose().tanh().transpose()
        elif op == "max":
            vals[out] = a.max(args[1], keepdims=args[2])
        elif op == "relu":
            vals[out] = a.relu()
        elif op == "addmax":
            m, axis, keep = vals[args[1]], args[2], args[3]
            shape = vals[args[0]].data.shape if is_numpy else vals[args[0]].shape
            if not keep:  # put the reduced axis back: (n,) -> (1, n), (m,) -> (m, 1)
                m = m.reshape((1, shape[1]) if axis == 0 else (shape[0], 1))
            vals[out] = a + m.expand(shape)
        elif op == "reduce":
            r = args[1]
            vals[out] = a.sum(0) if r == 0 else (a.sum(1) if r == 1 else a)
    return vals["out"], L


def device_grads(spec, dev):
    from ormi_amd import Tensor

    def mk(name, arr):
        return Tensor(arr, dev, requires_grad=name not in ("I",))

    out, L = run(spec, mk, False)
    loss = (out * Tensor(spec["w"], dev)).sum()
    loss.backward()
    grads = {k: t.grad.numpy() for k, t in L.items() if t.requires_grad and t.grad is not None}
    loss.zero_grad_graph()
    return grads


def numpy_grads(spec):
    out, L = run(spec, lambda name, arr: V(arr), True)
    loss = (out * V(spec["w"])).sum()
    loss.backward()
    return {k: v.grad for k, v in L.items() if k != "I" and v.grad is not None}


def check(spec, got):
    want = numpy_grads(spec)
    assert set(got) == set(want), (sorted(got), sorted(want))
    for k, g in got.items():
        w = want[k]
        assert g.shape == w.shape, k
        scale = np.abs(w).max()
        if scale == 0:
            assert np.all(g == 0), k
            continue
        rel = np.linalg.norm(g.astype(np.float64) - w) / np.linalg.norm(w)
        assert rel <= 1e-4, (spec["seed"], k, rel)
        assert np.all(np.abs(g - w) <= 1e-3 * scale), (spec["seed"], k)


def test_numpy_autograd_matches_finite_differences():
    """The reference itself: central differences in float64 on a small case."""
    spec = make_case(3)
    want = numpy_grads(spec)
    rng = np.random.default_rng(0)
    for name in ("X", "W", "b", "s", "R"):
        arr = spec["leaves"][name]
        for _ in range(4):
            idx = tuple(int(rng.integers(0, d)) for d in arr.shape)
            h = 1e-6

            def f(delta):
                leaves = {k: v.astype(np.float64).copy() for k, v in spec["leaves"].items()}
                leaves[name][idx] += delta
                sp = dict(spec, leaves=leaves)
                out, _ = run(sp, lambda nm, a: V(a), True)
                return float((out * V(spec["w"])).sum().data)
            fd = (f(h) - f(-h)) / (2 * h)
            assert abs(fd - want[name][idx]) <= 1e-5 * (1 + abs(fd)), (name, idx, fd, want[name][idx])


@pytest.mark.parametrize("seed", range(40))
def test_oracle_gradients_match_independent_autograd(cpu, seed):
    spec = make_case(seed)
    check(spec, device_grads(spec, cpu))


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(40))
def test_hip_gradients_match_independent_autograd(hip, seed):
    spec = make_case(seed)
    check(spec, device_grads(spec, hip))
