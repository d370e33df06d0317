"""Loads the native module. There is no Python fallback: without the built
extension the package does not import."""
try:
    from . import ormi_backend  # noqa: F401
except ImportError as e:  # pragma: no cover - exercised only on an unbuilt tree
    raise ImportError(
        "ormi_amd: the native module is not built. Run `python -m ormi_amd._build` "
        "(needs hipcc from ROCm and g++)."
    ) from e

__all__ = ["ormi_backend"]
