"""Tensor: the Python face of the lazy graph.

Same constructor, operators, views, realize/numpy/backward/zero_grad as
ormi_core.Tensor (reference ormi-core/src/ormi_core/tensor.py:10-190). Additive:
the "hip" device, a dtype argument for leaves, and element-wise / reduction
methods for the ops the reference lacks (relu, tanh, sigmoid, gelu, sum, mean,
max, argmax, astype).
"""
from __future__ import annotations

import math

import numpy as np
from numpy.lib.stride_tricks import as_strided

from ._ext import ormi_backend
from .exceptions import raise_device_mismatch

OpEnum = ormi_backend.OpEnum
DeviceEnum = ormi_backend.DeviceEnum
Device = ormi_backend.Device
Node = ormi_backend.Node

_DEVICE_STRINGS = {"cpu": DeviceEnum.CPU, "cuda": DeviceEnum.CUDA, "hip": DeviceEnum.HIP}


# One canonical Device object per (type, id), kept for the process: tensors on
# the same device share it, so device checks and the scalar-leaf cache can
# compare identities. _CANONICAL_IDS holds only these never-freed objects.
_CANONICAL: dict = {}
_CANONICAL_IDS: dict = {}


def _canonical(device: Device) -> Device:
    if id(device) in _CANONICAL_IDS:
        return device
    key = (int(device.type), device.id)
    canon = _CANONICAL.get(key)
    if canon is None:
        canon = _CANONICAL[key] = device
        _CANONICAL_IDS[id(device)] = device
    return canon


def _parse_device(device) -> Device:
    if device is None:
        return _canonical(Device(DeviceEnum.CPU, 0))
    if isinstance(device, str):
        name, _, idx = device.lower().partition(":")
        if name not in _DEVICE_STRINGS:
            raise_device_mismatch(msg="Unsupported string backend", got=device)
        return _canonical(Device(_DEVICE_STRINGS[name], int(idx) if idx else 0))
    if isinstance(device, DeviceEnum):
        return _canonical(Device(device, 0))
    if isinstance(device, Device):
        return _canonical(device)
    raise_device_mismatch(msg="Device argument is of invalid type.", got=type(device))


_SCALAR_LEAVES: dict = {}


def _scalar_leaf(value: float, device: Device) -> Node:
    """0-d constant leaf for a Python scalar operand, as Ormi makes one per use
    (reference tensor.py:80-85), but created once per (device, value): leaves are
    never written after creation, so sharing them is invisible to results and
    saves a host-to-device copy on every operation with a literal."""
    # device is canonical (one object per device, hashed by identity);
    # -0.0 == 0.0 as a float, so a zero's key carries its sign.
    key = (device, value) if value != 0.0 else (device, value, math.copysign(1.0, value))
    node = _SCALAR_LEAVES.get(key)
    if node is None:
        if len(_SCALAR_LEAVES) >= 4096:
            _SCALAR_LEAVES.clear()
        buf = ormi_backend.numpy_to_buffer(np.array(value, dtype=np.float32), device.type)
        node = Node(buf, False, device)
        _SCALAR_LEAVES[key] = node
    return node


_binary_node = ormi_backend._binary
_unary_node = ormi_backend._unary
_ADD, _SUB, _MUL, _DIV = OpEnum.ADD, OpEnum.SUB, OpEnum.MUL, OpEnum.DIV


class Tensor:
    # Two attributes, no per-instance dict: every graph op creates one Tensor.
    __slots__ = ("device", "_node")

    def __init__(self, data=None, device=None, requires_grad: bool = False, _node: Node | None = None,
                 dtype: str | None = None):
        self.device = _parse_device(device)
        if _node is not None:
            self._node = _node
        elif data is not None:
            if not isinstance(data, np.ndarray):
                data = np.array(data, dtype=np.int64 if dtype == "int64" else np.float32)
            buffer = ormi_backend.numpy_to_buffer(data, self.device.type, dtype)
            self._node = Node(buffer, requires_grad, self.device)
        else:
            self._node = None

    @classmethod
    def _wrap(cls, node: Node, device: Device) -> "Tensor":
        """A Tensor over an existing node with an already-parsed device (the
        constructor's work minus argument parsing; every op result uses it)."""
        t = _new_tensor(cls)
        t.device = device
        t._node = node
        return t

    # ------------------------------------------------------------ properties
    @property
    def op(self):
        return self._node.op if self._node else OpEnum.LEAF

    @property
    def requires_grad(self) -> bool:
        return self._node.requires_grad if self._node else False

    @property
    def shape(self):
        return tuple(self._node.shape) if self._node else None

    @property
    def dtype(self) -> str | None:
        return self._node.dtype if self._node else None

    @property
    def grad(self):
        node = self._node
        g = node.grad if node is not None else None
        if g is None:
            return None
        t = _new_tensor(Tensor)
        t.device = self.device
        t._node = g
        return t

    # ------------------------------------------------------------- operators
    def _ensure_tensor(self, other) -> "Tensor":
        if isinstance(other, Tensor):
            if other.device is not self.device and self.device.type != other.device.type:
                raise_device_mismatch(msg="Cannot mix devices in operation.", got=other.device.type)
            return other
        if isinstance(other, (int, float)) and not isinstance(other, bool):
            return Tensor._wrap(_scalar_leaf(float(other), self.device), self.device)
        return Tensor(data=other, device=self.device)

    def _binary(self, op, a: "Tensor", b: "Tensor") -> "Tensor":
        t = _new_tensor(Tensor)
        t.device = self.device
        t._node = _binary_node(op, a._node, b._node)
        return t

    def _unary(self, op) -> "Tensor":
        t = _new_tensor(Tensor)
        t.device = self.device
        t._node = _unary_node(op, self._node)
        return t

    def _other_node(self, other) -> Node:
        """The node of a right operand: a Tensor on this device (the common case
        first), a Python scalar (a cached 0-d leaf), or array data."""
        if type(other) is Tensor and other.device is self.device:
            return other._node
        if type(other) is float or type(other) is int:
            return _scalar_leaf(float(other), self.device)
        return self._ensure_tensor(other)._node

    def __add__(self, other):
        t = _new_tensor(Tensor)
        t.device = self.device
        t._node = _binary_node(_ADD, self._node, self._other_node(other))
        return t

    def __sub__(self, other):
        t = _new_tensor(Tensor)
        t.device = self.device
        t._node = _binary_node(_SUB, self._node, self._other_node(other))
        return t

    def __mul__(self, other):
        t = _new_tensor(Tensor)
        t.device = self.device
        t._node = _binary_node(_MUL, self._node, self._other_node(other))
        return t

    def __truediv__(self, other):
        t = _new_tensor(Tensor)
        t.device = self.device
        t._node = _binary_node(_DIV, self._node, self._other_node(other))
        return t

    def __pow__(self, power):
        return self._binary(OpEnum.POW, self, self._ensure_tensor(power))

    def __matmul__(self, other):
        if not isinstance(other, Tensor):
            raise TypeError("Matmul requires both operands to be Tensors.")
        if other.device is not self.device and self.device.type != other.device.type:
            raise_device_mismatch(msg="Cannot perform MATMUL across different devices", got=other.device.type)
        return self._binary(OpEnum.MATMUL, self, other)

    def __neg__(self):
        return self._unary(OpEnum.NEG)

    def __radd__(self, other):
        return self + other

    def __rmul__(self, other):
        return self * other

    def __rsub__(self, other):
        return self._binary(OpEnum.SUB, self._ensure_tensor(other), self)

    def __rtruediv__(self, other):
        return self._binary(OpEnum.DIV, self._ensure_tensor(other), self)

    # ------------------------------------------------ element-wise (additive)
    def exp(self):
        return self._unary(OpEnum.EXP)

    def log(self):
        return self._unary(OpEnum.LOG)

    def sin(self):
        return self._unary(OpEnum.SIN)

    def cos(self):
        return self._unary(OpEnum.COS)

    def relu(self):
        return self._unary(OpEnum.RELU)

    def tanh(self):
        return self._unary(OpEnum.TANH)

    def sigmoid(self):
        return self._unary(OpEnum.SIGMOID)

    def gelu(self):
        return self._unary(OpEnum.GELU)

    def astype(self, dtype: str) -> "Tensor":
        return Tensor._wrap(ormi_backend.cast(self._node, dtype), self.device)

    # ---------------------------------------------------- reductions (additive)
    @staticmethod
    def _axes(axis) -> list[int]:
        if axis is None:
            return []
        if isinstance(axis, int):
            return [axis]
        return list(axis)

    def sum(self, axis=None, keepdims: bool = False) -> "Tensor":
        return Tensor._wrap(ormi_backend.sum(self._node, self._axes(axis), keepdims), self.device)

    def max(self, axis=None, keepdims: bool = False) -> "Tensor":
        return Tensor._wrap(ormi_backend.max(self._node, self._axes(axis), keepdims), self.device)

    def argmax(self, axis: int | None = None, keepdims: bool = False) -> "Tensor":
        return Tensor._wrap(ormi_backend.argmax(self._node, self._axes(axis), keepdims), self.device)

    def mean(self, axis=None, keepdims: bool = False) -> "Tensor":
        """sum * (1/N), N = number of reduced elements (exact scaling for powers of two).
        An empty reduced range gives NaN (0 * inf), as numpy's mean does."""
        axes = self._axes(axis)
        shape = self.shape
        reduced = range(len(shape)) if not axes else [a % len(shape) for a in axes]
        n = 1
        for a in set(reduced):
            n *= shape[a]
        return self.sum(axis, keepdims) * (1.0 / n if n else math.inf)

    # ------------------------------------------------------------------ views
    def reshape(self, shape) -> "Tensor":
        return Tensor._wrap(ormi_backend.reshape(self._node, list(shape)), self.device)

    def transpose(self, axes=None) -> "Tensor":
        if axes is None:
            axes = tuple(reversed(range(len(self.shape))))
        return Tensor._wrap(ormi_backend.transpose(self._node, list(axes)), self.device)

    def expand(self, shape) -> "Tensor":
        return Tensor._wrap(ormi_backend.expand(self._node, list(shape)), self.device)

    @property
    def T(self) -> "Tensor":
        return self.transpose()

    # --------------------------------------------------------------- realize
    def realize(self) -> "Tensor":
        if self._node and self._node.is_realized:
            return self
        ormi_backend.execute_graph(self._node)
        return self

    def numpy(self) -> np.ndarray:
        self.realize()
        if not self._node or not self._node.is_realized:
            raise RuntimeError("Cannot fetch an unrealized tensor.")
        raw = ormi_backend.buffer_to_numpy(self._node.data)
        byte_strides = tuple(s * raw.itemsize for s in self._node.view.strides)
        return as_strided(raw, shape=self.shape, strides=byte_strides)

    def backward(self):
        if not self.requires_grad:
            raise RuntimeError("Cannot call backward() on a tensor that does not require gradients.")
        ormi_backend.compute_gradients(self._node)

    def zero_grad(self):
        node = self._node
        if node is not None:
            node._clear_grad()

    def zero_grad_graph(self):
        if self._node:
            ormi_backend.zero_grad_graph(self._node)

    def __repr__(self):
        state = "realized" if (self._node and self._node.is_realized) else "lazy"
        return f"Tensor(op={self.op.name}, shape={self.shape}, state={state}, device={self.device.type.name})"


_new_tensor = object.__new__


def realize_all(*tensors: Tensor) -> None:
    """Realize several tensors together. On the HIP device, element-wise roots
    of the same shape (for example the gradients of one backward pass, or the
    updated parameters of an SGD step) become one multi-output kernel that reads
    each shared input once; other tensors are realized one by one, in order."""
    nodes = [t._node for t in tensors if t is not None and t._node is not None]
    ormi_backend.realize_all(nodes)

