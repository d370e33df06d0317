"""Error types of the Python API (same names and messages as ormi_core.exceptions)."""


class OrmiError(Exception):
    pass


class DeviceMismatchError(OrmiError):
    pass


class ShapeMismatchError(OrmiError):
    pass


def raise_device_mismatch(msg: str, got, expected=None) -> None:
    err = f'{msg} | Got: "{got}"'
    if expected:
        err += f' | Expected: "{expected}"'
    raise DeviceMismatchError(err)


def raise_shape_error(msg: str, shape_a: tuple, shape_b: tuple) -> None:
    raise ShapeMismatchError(f"{msg} | Shape A: {shape_a}, Shape B: {shape_b}")
