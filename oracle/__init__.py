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
