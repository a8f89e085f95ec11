"""BarracudaError and its variants, mirroring crates/barracuda/src/error.rs:14-130.

Each C-ABI status code maps onto one variant (include/barracuda_hip.h).
"""
from __future__ import annotations


class BarracudaError(Exception):
    """Base of every error the op API returns (error.rs:17 BarracudaError)."""


class DeviceError(BarracudaError):
    """error.rs Device(String): device initialisation / runtime failure."""

    def __init__(self, msg: str):
        super().__init__(f"Device error: {msg}")


class DeviceNotAvailable(BarracudaError):
    """error.rs DeviceNotAvailable{device, reason} (:92-99): no HIP device, or
    the requested ordinal is not present."""

    def __init__(self, device: str, reason: str):
        self.device = device
        self.reason = reason
        super().__init__(f"Device not available: {device} - {reason}")


class DeviceLost(BarracudaError):
    """error.rs DeviceLost(String) (:52-59): the context can run no more work
    (a kernel fault, an uncorrectable ECC error).  Retriable on a fresh
    device, as the reference documents."""

    def __init__(self, msg: str):
        super().__init__(f"GPU device lost: {msg}")


class ShapeMismatch(BarracudaError):
    """error.rs ShapeMismatch{expected, actual} (:238)."""

    def __init__(self, expected, actual):
        self.expected = list(expected)
        self.actual = list(actual)
        super().__init__(f"Shape mismatch: expected {self.expected}, got {self.actual}")


class InvalidShape(BarracudaError):
    """error.rs InvalidShape{expected, actual} (:31-38, constructor :275)."""

    def __init__(self, expected, actual):
        self.expected = list(expected)
        self.actual = list(actual)
        super().__init__(f"Invalid shape: expected {self.expected}, got {self.actual}")


class InvalidOperation(BarracudaError):
    """error.rs InvalidOperation{op, reason} (:243)."""

    def __init__(self, op: str, reason: str):
        self.op = op
        self.reason = reason
        super().__init__(f"Invalid operation: {op} - {reason}")


class InvalidInput(BarracudaError):
    """error.rs InvalidInput{message} (:187)."""

    def __init__(self, message: str):
        self.message = message
        super().__init__(f"Invalid input: {message}")


class OutOfMemory(BarracudaError):
    """error.rs OutOfMemory(String)."""

    def __init__(self, msg: str):
        super().__init__(f"Out of memory: {msg}")


class ExecutionError(BarracudaError):
    """error.rs ExecutionError{message} (:230 execution_failed)."""

    def __init__(self, message: str):
        super().__init__(f"Execution error: {message}")


class CastOverflow(BarracudaError):
    """error.rs CastOverflow{from_type, to_type, value_description} (:143-152), raised by
    cast.rs:31-37 usize_as_u32."""

    def __init__(self, from_type: str, to_type: str, value_description: str):
        self.from_type, self.to_type = from_type, to_type
        self.value_description = value_description
        super().__init__(f"Cast overflow: {from_type} → {to_type} ({value_description})")


class UnsupportedOperation(BarracudaError):
    """error.rs UnsupportedOperation{op, device}."""

    def __init__(self, op: str, device: str):
        super().__init__(f"Operation not supported on device: {op} on {device}")


def from_status(status: int, msg: str, op: str = "op", device: str = "hip"):
    """Map a bch_status onto the matching BarracudaError variant."""
    from . import _native as N

    if status == N.BCH_E_INVALID:
        return InvalidInput(msg)
    if status == N.BCH_E_SHAPE:
        return InvalidOperation(op, f"shape/dimension mismatch: {msg}")
    if status == N.BCH_E_NO_DEVICE:
        return DeviceNotAvailable(device, msg)
    if status == N.BCH_E_DEVICE_LOST:
        return DeviceLost(msg)
    if status == N.BCH_E_OOM:
        return OutOfMemory(msg)
    if status == N.BCH_E_LAUNCH:
        return ExecutionError(msg)
    if status == N.BCH_E_UNSUPPORTED:
        return UnsupportedOperation(op, f"{device}: {msg}")
    return DeviceError(msg)
