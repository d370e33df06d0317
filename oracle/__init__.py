"""TEST INFRASTRUCTURE — the CPU oracle.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this
package, and only as the checker / reported baseline. It restates Ormi's CPU
backend in C++ (cpu_backend/cpu_backend.cpp, each function citing the reference
file it follows) and registers it as the "cpu" device of the already-loaded
core, so the same graph can be realized on "cpu" (oracle) and "hip" (product).
The product path never imports it.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

_LIB = Path(__file__).resolve().parent / "_build" / "libormi_cpu_oracle.so"
_handle = None


def load() -> None:
    """Register the CPU oracle device (idempotent)."""
    global _handle
    if _handle is not None:
        return
    import ormi_amd  # noqa: F401  loads libormi_core.so first

    if not _LIB.exists():
        raise ImportError(f"CPU oracle not built ({_LIB}); run `python -m ormi_amd._build`.")
    _handle = ctypes.CDLL(str(_LIB), mode=ctypes.RTLD_GLOBAL)
    assert _handle.ormi_oracle_loaded() == 1


# ----------------------------------------------------------------------------
# The reference's own CPU path (oracle/_ref/libormi_ref.so, built from
# /root/reference by oracle/Makefile.ref with oracle/ref_driver.cpp). It is
# built in the container that holds the reference sources and, like every
# built library, travels with the tree: the GPU box runs the prebuilt file
# (bench.py times it there as C3_reference). Loaded RTLD_LOCAL: its symbols
# never mix with the core's.
_REF_DIR = Path(__file__).resolve().parent / "_ref"
_REF_LIB = _REF_DIR / "libormi_ref.so"
_ref_handle = None

REF_OPS = {"NEG": 0, "EXP": 1, "LOG": 2, "SIN": 3, "COS": 4, "ADD": 5, "SUB": 6, "MUL": 7, "DIV": 8, "POW": 9,
           "SUM": 10, "TRANSPOSE": 11, "RESHAPE": 12, "EXPAND": 13, "MATMUL": 14}
REF_DEVICES = {"cpu": 0, "hip": 2}  # DeviceEnum values (HIP as the maintainer's edit numbers it)


class _RefLeaf(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("ndim", ctypes.c_int), ("shape", ctypes.c_int * 8),
                ("requires_grad", ctypes.c_int), ("numel", ctypes.c_longlong), ("has_strides", ctypes.c_int),
                ("strides", ctypes.c_int * 8)]


class _RefOp(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int), ("a", ctypes.c_int), ("b", ctypes.c_int), ("nattr", ctypes.c_int),
                ("attr", ctypes.c_int * 8), ("keepdims", ctypes.c_int)]


def ref_available() -> bool:
    return _REF_LIB.exists()


def load_ref_library(path: Path):
    """dlopen a library built from oracle/ref_driver.cpp (lazy binding: the two
    CUDA-device functions the reference declares, cuda::execute_jit and
    get_cuda_allocator, stay unresolved; no other device calls them)."""
    if not path.exists():
        raise ImportError(f"reference library not built ({path}); run `make -f oracle/Makefile.ref`.")
    h = ctypes.CDLL(str(path), mode=os.RTLD_LAZY | os.RTLD_LOCAL)
    h.ref_run.restype = ctypes.c_int
    h.ref_device_available.restype = ctypes.c_int
    return h


def ref_device_available(handle, device: str):
    """(available, message): whether the library's get_allocator(device) can be
    made, probed as the reference's test fixture does."""
    err = ctypes.create_string_buffer(512)
    ok = handle.ref_device_available(REF_DEVICES[device], err, 512)
    return bool(ok), err.value.decode()


def ref_call(handle, device: str, leaves, ops, outputs, grad_root: int = -1, capacity: int = 0):
    """Run a program through a driver library's execute_graph / compute_gradients
    on `device` ("cpu" or "hip"). See ref_run for the arguments; capacity is
    the room for each output in elements (default 64x the largest leaf)."""
    import numpy as np

    keep, views = [], []
    for leaf in leaves:
        a = leaf[0]
        if len(leaf) > 2:  # (buffer, requires_grad, (shape, strides)): a strided view over a flat buffer
            keep.append(np.ascontiguousarray(a, dtype=np.float32).reshape(-1))
            views.append(leaf[2])
        else:
            keep.append(np.ascontiguousarray(a, dtype=np.float32))
            views.append(None)
    L = (_RefLeaf * max(1, len(leaves)))()
    for i, (arr, leaf, view) in enumerate(zip(keep, leaves, views)):
        L[i].data, L[i].requires_grad = arr.ctypes.data, int(leaf[1])
        shape = arr.shape if view is None else tuple(view[0])
        L[i].ndim = len(shape)
        for d, e in enumerate(shape):
            L[i].shape[d] = e
        if view is not None:
            L[i].numel, L[i].has_strides = max(1, arr.size), 1
            for d, st in enumerate(view[1]):
                L[i].strides[d] = st
    O = (_RefOp * max(1, len(ops)))()
    for k, (name, a, b, attr, keepdims) in enumerate(ops):
        O[k].op, O[k].a, O[k].b, O[k].nattr, O[k].keepdims = REF_OPS[name], a, b, len(attr), int(keepdims)
        for d, x in enumerate(attr):
            O[k].attr[d] = x
    cap = capacity or max([a.size for a in keep] + [1]) * 64
    bufs = [np.empty(cap, np.float32) for _ in outputs]
    ptrs = (ctypes.c_void_p * len(outputs))(*[b.ctypes.data for b in bufs])
    caps = (ctypes.c_longlong * len(outputs))(*[cap] * len(outputs))
    ids = (ctypes.c_int * len(outputs))(*outputs)
    ndim = (ctypes.c_int * len(outputs))()
    shapes = (ctypes.c_int * (8 * len(outputs)))()
    err = ctypes.create_string_buffer(512)
    rc = handle.ref_run(REF_DEVICES[device], len(leaves), L, len(ops), O, grad_root, len(outputs), ids, ptrs, caps,
                        ndim, shapes, err, 512)
    if rc != 0:
        raise RuntimeError("reference: " + err.value.decode())
    res = []
    for o, b in enumerate(bufs):
        if ndim[o] < 0:  # a leaf the gradient does not reach
            res.append(None)
            continue
        shape = tuple(shapes[8 * o + d] for d in range(ndim[o]))
        res.append(b[: int(np.prod(shape, dtype=np.int64))].reshape(shape).copy())
    return res


def ref_run(leaves, ops, outputs, grad_root: int = -1):
    """Run a program through the reference's execute_graph / compute_gradients
    on its CPU device.

    leaves: [(float32 array, requires_grad)] (or (flat buffer, requires_grad,
    (shape, strides)) for a strided view over a buffer); ops: [(name, a, b, attr, keepdims)]
    over value ids (leaves first, then one value per op); outputs: value ids,
    or -1 - i for leaf i's gradient. Returns one float32 array per output
    (None for a leaf the gradient does not reach)."""
    global _ref_handle
    if _ref_handle is None:
        _ref_handle = load_ref_library(_REF_LIB)
    return ref_call(_ref_handle, "cpu", leaves, ops, outputs, grad_root)
