"""Float64 reference of one C5 training step, and per-operation bounds.

The step is the MLP of the C5 config: H1 = gelu(X W1), H2 = gelu(H1 W2),
Y = H2 W3, loss = sum((Y - T)^2) * 2^-20, then the backward autograd builds
(reference csrc/core/ops/blas/matmul.cpp:71-135 for the matmul adjoints,
csrc/core/autograd.cpp:24-47 for the reverse pass) and SGD W - lr * dW.

A componentwise worst-case bound carried through the whole step is useless:
absolute values lose the sign cancellation of every product, and for dW1 the
bound comes out about 1e5 times the gradient itself. The step is therefore
checked link by link: every operation's device output against the float64
value of that operation on the device's own inputs, within
  * a length-K fp32 product: 2 K eps32 (|A| |B|), the bound every test of this
    suite uses for a GEMM (any summation order);
  * gelu / gelu': C_ACT ulp of (|f| + |z|), the formula's roundings plus a
    few-ulp erf; the |z| term covers the cancellation in 1 + erf(z / sqrt 2);
and end to end, normwise, against the float64 step (mlp_step_f64).
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

EPS32 = float(np.finfo(np.float32).eps)
U = EPS32 / 2
C_ACT = 8.0
SQRT_HALF = 1.0 / math.sqrt(2.0)
INV_SQRT_2PI = 1.0 / math.sqrt(2.0 * math.pi)


def gelu(z):
    return 0.5 * z * (1.0 + erf(z * SQRT_HALF))


def gelu_grad(z):
    return 0.5 * (1.0 + erf(z * SQRT_HALF)) + z * INV_SQRT_2PI * np.exp(-0.5 * z * z)


def mlp_step_f64(X, T, Ws, lr=1e-3):
    """The exact step in float64: loss, [dW1, dW2, dW3], updated weights."""
    X = X.astype(np.float64)
    T = T.astype(np.float64)
    W = [w.astype(np.float64) for w in Ws]
    c = 1.0 / (X.shape[0] * T.shape[1])
    Z1 = X @ W[0]
    H1 = gelu(Z1)
    Z2 = H1 @ W[1]
    H2 = gelu(Z2)
    D = H2 @ W[2] - T
    loss = float((D * D).sum() * c)
    dY = 2 * c * D
    dW3 = H2.T @ dY
    dZ2 = (dY @ W[2].T) * gelu_grad(Z2)
    dW2 = H1.T @ dZ2
    dZ1 = (dZ2 @ W[1].T) * gelu_grad(Z1)
    dW1 = X.T @ dZ1
    grads = [dW1, dW2, dW3]
    return loss, grads, [w - g * lr for w, g in zip(W, grads)]


def gemm_excess(got, a, b):
    """max over entries of |got - a b| / (2 K eps32 |a||b|), a and b the device
    operands as float64 (<= 1 passes)."""
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    bound = 2 * a.shape[1] * EPS32 * (np.abs(a64) @ np.abs(b64))
    err = np.abs(got.astype(np.float64) - a64 @ b64)
    return float(np.max(err / np.maximum(bound, np.finfo(np.float64).tiny)))


def act_excess(got, z, fn):
    """max of |got - fn(z)| / (C_ACT u (|fn(z)| + |z|)) with z the device input."""
    z64 = z.astype(np.float64)
    want = fn(z64)
    bound = C_ACT * U * (np.abs(want) + np.abs(z64))
    return float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(bound, np.finfo(np.float64).tiny)))


def normwise(got, want):
    return float(np.linalg.norm(got.astype(np.float64) - want) / np.linalg.norm(want))
