"""A float64 reverse-mode autograd over numpy, independent of the graph core.

The oracle and the HIP device share libormi_core.so (shape rules, adjoints,
autograd), so a mistake there would be common to both. This module restates the
derivatives from the mathematics instead: each op records its inputs and a
function from the output's gradient to the inputs' gradients; broadcast inputs
get their gradient summed back over the broadcast axes (numpy's rules). It is
test infrastructure only.
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

INV_SQRT_2PI = 1.0 / math.sqrt(2.0 * math.pi)


def _unbroadcast(g: np.ndarray, shape) -> np.ndarray:
    shape = tuple(shape)
    while g.ndim > len(shape):
        g = g.sum(axis=0)
    for i, s in enumerate(shape):
        if s == 1 and g.shape[i] != 1:
            g = g.sum(axis=i, keepdims=True)
    return g.reshape(shape)


class V:
    """A value in the tape: data (float64), parents and the backward rule."""

    def __init__(self, data, parents=(), back=None):
        self.data = np.asarray(data, dtype=np.float64)
        self.parents = parents
        self.back = back
        self.grad = None

    # ------------------------------------------------------------ element-wise
    def _bin(self, other, f, df):
        o = other if isinstance(other, V) else V(np.float64(other))
        out = f(self.data, o.data)

        def back(g):
            ga, gb = df(self.data, o.data, out, g)
            return [_unbroadcast(ga, self.data.shape), _unbroadcast(gb, o.data.shape)]
        return V(out, (self, o), back)

    def __add__(self, o):
        return self._bin(o, lambda a, b: a + b, lambda a, b, y, g: (g, g))

    def __sub__(self, o):
        return self._bin(o, lambda a, b: a - b, lambda a, b, y, g: (g, -g))

    def __mul__(self, o):
        return self._bin(o, lambda a, b: a * b, lambda a, b, y, g: (g * b, g * a))

    def __truediv__(self, o):
        return self._bin(o, lambda a, b: a / b, lambda a, b, y, g: (g / b, -g * a / (b * b)))

    def __pow__(self, o):
        return self._bin(o, lambda a, b: a ** b,
                         lambda a, b, y, g: (g * b * a ** (b - 1.0), g * y * np.log(np.where(a > 0, a, 1.0))))

    def _un(self, f, df):
        out = f(self.data)
        return V(out, (self,), lambda g: [g * df(self.data, out)])

    def __neg__(self):
        return self._un(lambda a: -a, lambda a, y: -np.ones_like(a))

    def exp(self):
        return self._un(np.exp, lambda a, y: y)

    def log(self):
        return self._un(np.log, lambda a, y: 1.0 / a)

    def sin(self):
        return self._un(np.sin, lambda a, y: np.cos(a))

    def cos(self):
        return self._un(np.cos, lambda a, y: -np.sin(a))

    def tanh(self):
        return self._un(np.tanh, lambda a, y: 1.0 - y * y)

    def sigmoid(self):
        return self._un(lambda a: 1.0 / (1.0 + np.exp(-a)), lambda a, y: y * (1.0 - y))

    def relu(self):
        return self._un(lambda a: np.maximum(a, 0.0), lambda a, y: (a > 0).astype(np.float64))

    def gelu(self):
        return self._un(lambda a: 0.5 * a * (1.0 + erf(a / math.sqrt(2.0))),
                        lambda a, y: 0.5 * (1.0 + erf(a / math.sqrt(2.0))) + a * INV_SQRT_2PI * np.exp(-0.5 * a * a))

    # --------------------------------------------------------------- structure
    def __matmul__(self, o):
        out = self.data @ o.data

        def back(g):
            ga = g @ np.swapaxes(o.data, -1, -2)
            gb = np.swapaxes(self.data, -1, -2) @ g
            return [_unbroadcast(ga, self.data.shape), _unbroadcast(gb, o.data.shape)]
        return V(out, (self, o), back)

    def sum(self, axis=None, keepdims=False):
        out = self.data.sum(axis=axis, keepdims=keepdims)

        def back(g):
            if not keepdims and axis is not None:
                g = np.expand_dims(g, axis)
            return [np.broadcast_to(g, self.data.shape).copy()]
        return V(out, (self,), back)

    def max(self, axis=None, keepdims=False):
        out = self.data.max(axis=axis, keepdims=keepdims)

        def back(g):
            m = out if keepdims or axis is None else np.expand_dims(out, axis)
            gg = g if keepdims or axis is None else np.expand_dims(g, axis)
            return [np.broadcast_to(gg, self.data.shape) * (self.data == m)]
        return V(out, (self,), back)

    def transpose(self, axes=None):
        axes = tuple(reversed(range(self.data.ndim))) if axes is None else tuple(axes)
        inv = np.argsort(axes)
        return V(np.transpose(self.data, axes), (self,), lambda g: [np.transpose(g, inv)])

    def reshape(self, shape):
        return V(self.data.reshape(shape), (self,), lambda g: [g.reshape(self.data.shape)])

    def expand(self, shape):
        return V(np.broadcast_to(self.data, shape).copy(), (self,), lambda g: [_unbroadcast(g, self.data.shape)])

    # ---------------------------------------------------------------- backward
    def backward(self):
        order, seen = [], set()
        stack = [(self, False)]
        while stack:
            v, done = stack.pop()
            if done:
                order.append(v)
                continue
            if id(v) in seen:
                continue
            seen.add(id(v))
            stack.append((v, True))
            for p in v.parents:
                stack.append((p, False))
        self.grad = np.ones_like(self.data)
        for v in reversed(order):
            if v.back is None or v.grad is None:
                continue
            for p, g in zip(v.parents, v.back(v.grad)):
                p.grad = g if p.grad is None else p.grad + g


def run_program(leaves, ops, outputs, grad_root=-1):
    """A driver program (oracle.ref_call's format: leaves [(array,
    requires_grad)], ops [(name, a, b, attr, keepdims)], outputs as value ids or
    -1 - leaf for a leaf's gradient) evaluated in float64. Returns one float64
    array per output (None for a leaf the gradient does not reach)."""
    vals = [V(np.asarray(a, np.float64)) for a, *_ in leaves]
    un = {"NEG": V.__neg__, "EXP": V.exp, "LOG": V.log, "SIN": V.sin, "COS": V.cos}
    bi = {"ADD": V.__add__, "SUB": V.__sub__, "MUL": V.__mul__, "DIV": V.__truediv__, "POW": V.__pow__,
          "MATMUL": V.__matmul__}
    for name, a, b, attr, keepdims in ops:
        x = vals[a]
        if name in un:
            vals.append(un[name](x))
        elif name in bi:
            vals.append(bi[name](x, vals[b]))
        elif name == "SUM":
            vals.append(x.sum(axis=tuple(attr) if attr else None, keepdims=bool(keepdims)))
        elif name == "TRANSPOSE":
            vals.append(x.transpose(attr))
        elif name == "RESHAPE":
            vals.append(x.reshape(attr))
        elif name == "EXPAND":
            vals.append(x.expand(attr))
        else:
            raise ValueError(name)
    if grad_root >= 0:
        vals[grad_root].backward()
    res = []
    for o in outputs:
        if o >= 0:
            res.append(vals[o].data)
        else:
            g = vals[-1 - o].grad
            res.append(None if g is None or not leaves[-1 - o][1] else g)
    return res
