"""MI355X-native device for the Ormi lazy tensor / autograd engine.

`Tensor(..., device="hip")` builds lazy graphs exactly as Ormi's Tensor does;
realizing them runs fused hipRTC kernels, LDS/DPP reductions and MFMA GEMMs on
the GPU through libormi_hip.so (C ABI in include/ormi_hip.h).
"""
from ._ext import ormi_backend
from .tensor import Tensor, realize_all
from .exceptions import OrmiError, DeviceMismatchError, ShapeMismatchError

__version__ = "0.1.0"
__all__ = ["Tensor", "realize_all", "ormi_backend", "OrmiError", "DeviceMismatchError", "ShapeMismatchError"]
