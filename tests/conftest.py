"""Shared fixtures. `gpu` marks tests that need the MI355X (HIP device)."""
import ctypes
import re
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (the HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def ob():
    import ormi_amd

    return ormi_amd.ormi_backend


@pytest.fixture(scope="session")
def cpu(ob):
    """The CPU oracle device (test infrastructure)."""
    import oracle

    oracle.load()
    return "cpu"


@pytest.fixture(scope="session")
def hip(ob):
    """The HIP device. GPU tests fail (not skip) when it is missing, so a GPU run
    that silently lost the device cannot pass."""
    assert ob.hip_available(), "HIP device unavailable: these tests need the MI355X"
    return "hip"


@pytest.fixture(scope="session")
def cabi():
    """libormi_hip.so through ctypes, with argtypes from include/ormi_hip.h."""
    lib = ctypes.CDLL(str(ROOT / "ormi_amd" / "lib" / "libormi_hip.so"))
    lib.ormi_hip_last_error.restype = ctypes.c_char_p
    for name in ["ormi_hip_malloc"]:
        getattr(lib, name).argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    lib.ormi_hip_free.argtypes = [ctypes.c_void_p]
    lib.ormi_hip_memcpy_h2d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    lib.ormi_hip_memcpy_d2h.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    lib.ormi_hip_memcpy_d2d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    lib.ormi_hip_fill.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t]
    lib.ormi_hip_convert.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    lib.ormi_hip_rtc_compile_only.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                              ctypes.c_int, ctypes.POINTER(ctypes.c_size_t)]
    return lib


def map_tile_groups(ob) -> int:
    """Groups per map tile (256 threads x the planned unroll), from a plan."""
    from ormi_amd import Tensor

    plan = ob._plan_kernel((Tensor(np.zeros(4, np.float32), "cpu") * 2.0)._node)["plan"]
    return 256 * int(plan.split("unroll=")[1].split()[0])


def empty_tensor_cases(dev: str) -> dict:
    """Graphs over 0-length dims on `dev`: name -> numpy result, or the
    ("error", message) a reduction with no identity raises. numpy's rules: a
    0-length dim broadcasts against 1 to 0; sum over nothing is 0, mean NaN;
    max/argmax over nothing raise unless the result itself is empty; a K = 0
    product is zeros. Gradients flow through empty operands."""
    from ormi_amd import Tensor

    def T(shape, fill=0.0, **kw):
        return Tensor(np.full(shape, fill, np.float32), dev, **kw)

    cases = {
        "bcast_rows": lambda: T((0, 5)) + T((5,), 1.0),
        "bcast_cols": lambda: T((3, 0)) * T((3, 1), 2.0),
        "bcast_both": lambda: T((0, 1)) - T((1, 7), 1.0),
        "unary": lambda: T((4, 0)).tanh(),
        "sum_rows": lambda: T((0, 5)).sum(0),
        "sum_cols": lambda: T((0, 5)).sum(1),
        "sum_all": lambda: T((0, 5)).sum(),
        "sum_keep": lambda: T((2, 0, 3)).sum(1, keepdims=True),
        "mean_empty": lambda: T((0, 5)).mean(0),
        "max_kept_empty": lambda: T((0, 5)).max(1),
        "max_over_empty": lambda: T((0, 5)).max(0),
        "argmax_over_empty": lambda: T((3, 0)).argmax(1),
        "matmul_k0": lambda: T((3, 0)) @ T((0, 4)),
        "matmul_m0": lambda: T((0, 3), 1.0) @ T((3, 4), 1.0),
        "matmul_n0": lambda: T((3, 4), 1.0) @ T((4, 0)),
        "matmul_batched_k0": lambda: T((2, 3, 0)) @ T((2, 0, 5)),
    }
    out = {}
    for name, f in cases.items():
        try:
            out[name] = f().numpy()
        except RuntimeError as e:
            out[name] = ("error", str(e))
    a = T((0, 5), requires_grad=True)
    b = T((5,), 1.0, requires_grad=True)
    w = T((5, 3), 1.0, requires_grad=True)
    ((a * b) @ w).sum().backward()
    out["grad_a"], out["grad_b"], out["grad_w"] = a.grad.numpy(), b.grad.numpy(), w.grad.numpy()
    return out


def header_functions():
    text = (ROOT / "include" / "ormi_hip.h").read_text()
    return sorted(set(re.findall(r"\b(ormi_hip_\w+)\s*\(", text)))


def fp32_sum_tolerance(x: np.ndarray, axis) -> np.ndarray:
    """Bound for |fp32 sum (any order) - exact sum|: n * eps32 * sum|x| (Higham)."""
    n = x.size if axis is None else np.prod([x.shape[a] for a in np.atleast_1d(axis)])
    return n * np.finfo(np.float32).eps * np.abs(x.astype(np.float64)).sum(axis=axis)
