"""TensorError mirror of the reference's error enum (src/error.rs:7-71).

The Display formats are kept identical so callers matching on messages behave the same. Paths where
the reference panics (assert!/assert_eq!/expect) raise `Panic`, an AssertionError.
"""
from __future__ import annotations

from . import _lib


class TensorError(Exception):
    """Base of the reference's `TensorError` variants."""


class ShapeMismatch(TensorError):
    def __init__(self, operation: str, expected: str, got: str):
        self.operation, self.expected, self.got = operation, expected, got
        super().__init__(f"{operation}: shape mismatch, expected {expected}, got {got}")


class UnsupportedDimensions(TensorError):
    def __init__(self, operation: str, expected: str, got: list):
        self.operation, self.expected, self.got = operation, expected, list(got)
        super().__init__(f"{operation}: unsupported dimensions, expected {expected}, got {list(got)}")


class PrecisionMismatch(TensorError):
    def __init__(self, operation: str, expected: str, got: str):
        self.operation, self.expected, self.got = operation, expected, got
        super().__init__(f"{operation}: precision mismatch, expected {expected}, got {got}")


class InnerDimensionMismatch(TensorError):
    def __init__(self, operation: str, a_shape: list, b_shape: list):
        self.operation, self.a_shape, self.b_shape = operation, list(a_shape), list(b_shape)
        super().__init__(
            f"{operation}: inner dimensions don't match, A={list(a_shape)}, B={list(b_shape)}")


class EmptyTensor(TensorError):
    def __init__(self, operation: str):
        self.operation = operation
        super().__init__(f"{operation}: empty tensor not supported")


class InvalidValue(TensorError):
    def __init__(self, operation: str, message: str):
        self.operation, self.message = operation, message
        super().__init__(f"{operation}: {message}")


class Panic(AssertionError):
    """Where the reference panics (assert!, assert_eq!, expect)."""


class DeviceError(RuntimeError):
    """HIP runtime failure, allocation failure or missing device (reference panics on these)."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"[{_lib.status_name(status)}] {message}")


def check(status: int, operation: str = "") -> None:
    """Raises the mirror exception for a non-OK it_status, with the library's message."""
    if status == _lib.IT_OK:
        return
    msg = _lib.last_error()
    if status == _lib.IT_ERR_PRECISION:
        raise TensorError(msg)
    if status in (_lib.IT_ERR_INVALID, _lib.IT_ERR_NULL, _lib.IT_ERR_SHAPE, _lib.IT_ERR_DIMS,
                  _lib.IT_ERR_INNER_DIM):
        raise InvalidValue(operation or "irontensor", msg)
    raise DeviceError(status, msg)
