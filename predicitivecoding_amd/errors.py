"""Exceptions mirroring the reference's error behaviour on this path.

BatchedPcForward.cs:42-57 throws ArgumentNullException, ArgumentException and
ArgumentOutOfRangeException; Network.ExportGenerativeSnapshot throws
NotSupportedException (Network.cs:1334-1338); native failures surface as
DeviceException(code) with a DeviceStatus code (Interop/CudaStatus.cs:7-38).
"""
from __future__ import annotations

from enum import IntEnum


class DeviceStatus(IntEnum):
    Success = 0
    NotInitialized = 1
    NoDevice = 2
    OutOfMemory = 3
    InvalidValue = 4
    HipError = 5
    GemmError = 6
    CollectiveError = 7
    NotSupported = 8
    Unknown = 100


class ArgumentException(ValueError):
    pass


class ArgumentNullException(ArgumentException):
    pass


class ArgumentOutOfRangeException(ArgumentException):
    pass


class NotSupportedException(Exception):
    pass


class DeviceException(RuntimeError):
    """A native call returned a non-zero DeviceStatus."""

    def __init__(self, code: int, operation: str, detail: str = ""):
        try:
            name = DeviceStatus(code).name
        except ValueError:
            name = "Unknown"
        msg = f"Native device op '{operation}' failed with status {name} ({code})."
        if detail:
            msg += f" {detail}"
        super().__init__(msg)
        self.code = code
        self.operation = operation
