"""C5 at config size on the GPU: one MLP training step, batch 1024, layers
1024 -> 4096 -> 4096 -> 1024, GELU, MSE, SGD lr 1e-3, seed 4, through the
default fused path (SGD updates and activations in GEMM epilogues).

Checked link by link against float64 (bounds in mlp_ref.py): every GEMM of
the forward and of the backward autograd builds (reference
csrc/core/ops/blas/matmul.cpp:71-135, reverse pass csrc/core/autograd.cpp:24-47)
against the float64 product of its own device operands within 2 K eps32 |A||B|;
every gelu / gelu' within a few ulp; the loss gradient and the SGD updates
bit-exact against the same fp32 arithmetic; and end to end, the loss within
rtol 1e-5 and each weight gradient within a normwise 1e-4 of the float64 step.
"""
import math
import sys

import numpy as np
import pytest

from mlp_ref import U, C_ACT, act_excess, gelu, gelu_grad, gemm_excess, mlp_step_f64, normwise

def log(msg):
    print(f"[c5] {msg}", file=sys.stderr, flush=True)


def mul_act_excess(got, p, z, fn):
    """|got - p fn(z)| over (|p| C_ACT u (|fn(z)| + |z|) + u |got|): the product
    of a device operand p with an activation derivative of the device input z."""
    z64, p64 = z.astype(np.float64), p.astype(np.float64)
    f = fn(z64)
    bound = np.abs(p64) * C_ACT * U * (np.abs(f) + np.abs(z64)) + U * np.abs(got.astype(np.float64))
    err = np.abs(got.astype(np.float64) - p64 * f)
    return float(np.max(err / np.maximum(bound, np.finfo(np.float64).tiny)))


def run_step_and_check(ob, dev, batch, dims, seed=4, expect_fused=0):
    from ormi_amd import Tensor

    rng = np.random.default_rng(seed)
    X = rng.normal(0, 1, (batch, dims[0])).astype(np.float32)
    Tt = rng.normal(0, 1, (batch, dims[-1])).astype(np.float32)
    Ws = [rng.uniform(-math.sqrt(6 / i), math.sqrt(6 / i), (i, o)).astype(np.float32) for i, o in zip(dims, dims[1:])]
    lr = np.float32(1e-3)
    inv_n = 1.0 / (batch * dims[-1])
    c = np.float32(inv_n)

    log(f"{dev} step, batch {batch}, layers {dims}")
    before = ob.gemm_epilogue_count()
    ws = [Tensor(w, dev, requires_grad=True) for w in Ws]
    z1 = Tensor(X, dev) @ ws[0]
    h1 = z1.gelu()
    z2 = h1 @ ws[1]
    h2 = z2.gelu()
    y = h2 @ ws[2]
    d = y - Tensor(Tt, dev)
    loss = (d * d).sum() * inv_n
    loss.backward()
    new = [(w - w.grad * 1e-3).realize() for w in ws]  # the bench's step: updates first
    fused = ob.gemm_epilogue_count() - before
    assert fused >= expect_fused, f"expected the fused path (2 GELU + 2 dGELU + 3 SGD epilogues), got {fused}"
    new_np = [n.numpy() for n in new]
    loss_v = float(loss.numpy())
    # Device intermediates: buffers the step realized, or deterministic recomputations.
    Z1, H1, Z2, H2, Y = (t.numpy() for t in (z1, h1, z2, h2, y))
    dY, dH2, dZ2, dH1, dZ1 = (t.grad.numpy() for t in (y, h2, z2, h1, z1))
    dW = [w.grad.numpy() for w in ws]

    log("links: forward")
    assert gemm_excess(Z1, X, Ws[0]) <= 1
    assert act_excess(H1, Z1, gelu) <= 1
    assert gemm_excess(Z2, H1, Ws[1]) <= 1
    assert act_excess(H2, Z2, gelu) <= 1
    assert gemm_excess(Y, H2, Ws[2]) <= 1
    D = Y - Tt  # fp32, as the device subtracts
    want_loss = float((D.astype(np.float64) ** 2).sum()) * inv_n
    assert abs(loss_v - want_loss) <= 1e-5 * want_loss

    log("links: backward")
    # d(sum(d*d) c)/dY = c d + c d: exact in fp32 (c is a power of two)
    assert np.array_equal(dY, c * D + c * D)
    assert gemm_excess(dW[2], H2.T, dY) <= 1
    assert gemm_excess(dH2, dY, Ws[2].T) <= 1
    assert mul_act_excess(dZ2, dH2, Z2, gelu_grad) <= 1
    assert gemm_excess(dW[1], H1.T, dZ2) <= 1
    assert gemm_excess(dH1, dZ2, Ws[1].T) <= 1
    assert mul_act_excess(dZ1, dH1, Z1, gelu_grad) <= 1
    assert gemm_excess(dW[0], X.T, dZ1) <= 1
    for w, g, n in zip(Ws, dW, new_np):
        assert np.array_equal(n, w - g * lr)  # the SGD update (fused on HIP), bit for bit

    log("end to end vs the float64 step")
    loss64, grads64, _ = mlp_step_f64(X, Tt, Ws)
    assert abs(loss_v - loss64) <= 1e-5 * loss64
    for i, (g, g64) in enumerate(zip(dW, grads64)):
        assert normwise(g, g64) <= 1e-4, (i, normwise(g, g64))
    loss.zero_grad_graph()


@pytest.mark.gpu
def test_c5_mlp_step_full_size(ob, hip):
    run_step_and_check(ob, hip, 1024, [1024, 4096, 4096, 1024], expect_fused=7)


def test_c5_step_checks_on_the_oracle(ob, cpu):
    """The same link-by-link checks, on the CPU oracle at a small size."""
    run_step_and_check(ob, cpu, 64, [32, 128, 96, 48])
