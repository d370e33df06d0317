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
# /root/reference by oracle/Makefile.ref with oracle/ref_driver.cpp). Present
# only where the reference sources are (this container); tests that use it skip
# elsewhere. Loaded RTLD_LOCAL: its symbols never mix with the core's.
_REF_LIB = Path(__file__).resolve().parent / "_ref" / "libormi_ref.so"
_ref_handle = None

REF_OPS = {"NEG": 0, "EXP": 1, "LOG": 2, "SIN": 3, "COS": 4, "ADD": 5, "SUB": 6, "MUL": 7, "DIV": 8, "POW": 9,
           "SUM": 10, "TRANSPOSE": 11, "RESHAPE": 12, "EXPAND": 13}


class _RefLeaf(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("ndim", ctypes.c_int), ("shape", ctypes.c_int * 8),
                ("requires_grad", ctypes.c_int)]


class _RefOp(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int), ("a", ctypes.c_int), ("b", ctypes.c_int), ("nattr", ctypes.c_int),
                ("attr", ctypes.c_int * 8), ("keepdims", ctypes.c_int)]


def ref_available() -> bool:
    return _REF_LIB.exists()


def ref_run(leaves, ops, outputs, grad_root: int = -1):
    """Run a program through the reference's execute_graph / compute_gradients.

    leaves: [(float32 array, requires_grad)]; ops: [(name, a, b, attr, keepdims)]
    over value ids (leaves first, then one value per op); outputs: value ids,
    or -1 - i for leaf i's gradient. Returns one float32 array per output
    (None for a leaf the gradient does not reach)."""
    import numpy as np

    global _ref_handle
    if _ref_handle is None:
        if not _REF_LIB.exists():
            raise ImportError(f"reference CPU path not built ({_REF_LIB}); run `make -f oracle/Makefile.ref`.")
        # Lazy binding: the two CUDA-device functions the reference declares
        # (cuda::execute_jit, get_cuda_allocator) stay unresolved; the CPU
        # device never calls them.
        _ref_handle = ctypes.CDLL(str(_REF_LIB), mode=os.RTLD_LAZY | os.RTLD_LOCAL)
        _ref_handle.ref_run.restype = ctypes.c_int
    keep = [np.ascontiguousarray(a, dtype=np.float32) for a, _ in leaves]
    L = (_RefLeaf * max(1, len(leaves)))()
    for i, (arr, (_, rg)) in enumerate(zip(keep, leaves)):
        L[i].data, L[i].ndim, L[i].requires_grad = arr.ctypes.data, arr.ndim, int(rg)
        for d, e in enumerate(arr.shape):
            L[i].shape[d] = e
    O = (_RefOp * max(1, len(ops)))()
    for k, (name, a, b, attr, keepdims) in enumerate(ops):
        O[k].op, O[k].a, O[k].b, O[k].nattr, O[k].keepdims = REF_OPS[name], a, b, len(attr), int(keepdims)
        for d, x in enumerate(attr):
            O[k].attr[d] = x
    cap = max([a.size for a in keep] + [1]) * 64
    bufs = [np.empty(cap, np.float32) for _ in outputs]
    ptrs = (ctypes.c_void_p * len(outputs))(*[b.ctypes.data for b in bufs])
    caps = (ctypes.c_longlong * len(outputs))(*[cap] * len(outputs))
    ids = (ctypes.c_int * len(outputs))(*outputs)
    ndim = (ctypes.c_int * len(outputs))()
    shapes = (ctypes.c_int * (8 * len(outputs)))()
    err = ctypes.create_string_buffer(512)
    rc = _ref_handle.ref_run(len(leaves), L, len(ops), O, grad_root, len(outputs), ids, ptrs, caps, ndim, shapes,
                             err, 512)
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
