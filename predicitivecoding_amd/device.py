"""Device handles, device tensors, streams and tensor ops over the C ABI.

Host-side mirror of PredictiveCoding.Device: Device (Device.cs:20-39),
DeviceRuntime (DeviceRuntime.cs:14-83), DeviceTensor (DeviceTensor.cs:20-142),
CudaStreamManager (Streams/CudaStreamManager.cs:17-80) and TensorOps
(TensorOps.cs:17-104), with every device operation going through
libpcdevice_hip.  Unlike the reference there is no silent CPU fallback: a
call that needs the GPU raises DeviceException when none is present.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from enum import Enum

import numpy as np

from . import _native
from ._native import MEMCPY, call
from .errors import ArgumentException


class DeviceKind(Enum):
    Cpu = 0
    Cuda = 1
    CudaMulti = 2
    Metal = 3
    Rocm = 4


@dataclass(frozen=True)
class Device:
    kind: DeviceKind
    id: int = 0

    @staticmethod
    def cpu() -> "Device":
        return Device(DeviceKind.Cpu)

    @staticmethod
    def rocm(id: int = 0) -> "Device":
        return Device(DeviceKind.Rocm, id)

    @property
    def is_cpu(self) -> bool:
        return self.kind == DeviceKind.Cpu

    @property
    def is_gpu(self) -> bool:
        return not self.is_cpu

    def __str__(self) -> str:
        return "cpu" if self.is_cpu else f"{self.kind.name.lower()}:{self.id}"


class DeviceRuntime:
    """Lazy device probe (DeviceRuntime.cs:27-32,68-82)."""

    @staticmethod
    def device_count() -> int:
        n = ctypes.c_int(0)
        _native.lib().pcd_get_device_count(ctypes.byref(n))
        return n.value

    @staticmethod
    def available() -> bool:
        return DeviceRuntime.device_count() > 0

    @staticmethod
    def synchronize() -> None:
        call("pcd_device_synchronize")


class Stream:
    """A non-blocking HIP stream at the default priority."""

    def __init__(self, handle: int | None = None, owned: bool = True):
        if handle is None:
            h = ctypes.c_void_p()
            call("pcd_stream_create", ctypes.byref(h))
            handle = h.value
        self.handle = handle
        self._owned = owned and handle is not None

    def synchronize(self) -> None:
        call("pcd_stream_synchronize", self.handle)

    def close(self) -> None:
        if self._owned and self.handle:
            call("pcd_stream_destroy", self.handle)
        self.handle = None
        self._owned = False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        h = ctypes.c_void_p()
        call("pcd_event_create", ctypes.byref(h))
        self.handle = h.value

    def record(self, stream: Stream | None = None) -> None:
        call("pcd_event_record", self.handle, stream.handle if stream else None)

    def synchronize(self) -> None:
        call("pcd_event_synchronize", self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        call("pcd_event_elapsed_ms", ctypes.byref(ms), self.handle, end.handle)
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                _native.lib().pcd_event_destroy(self.handle)
        except Exception:
            pass


# float16 tensors hold fp16 GEMM operands; uint16 tensors hold raw bf16 bit
# patterns (numpy has no bfloat16).
_NP_DTYPES = {np.dtype(np.float32), np.dtype(np.float16), np.dtype(np.uint16), np.dtype(np.int32)}
_GEMM_FN = {np.dtype(np.float32): "pcd_gemm_f32", np.dtype(np.float16): "pcd_gemm_f16",
            np.dtype(np.uint16): "pcd_gemm_bf16"}


class DeviceTensor:
    """Row-major device buffer from the library's pooled allocator."""

    def __init__(self, shape, dtype=np.float32, stream: Stream | None = None):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        if self.dtype not in _NP_DTYPES:
            raise ArgumentException(f"unsupported dtype {self.dtype}")
        self.stream = stream
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        call("pcd_malloc_async", ctypes.byref(p), self.nbytes, self._s())
        self.ptr = p.value

    def _s(self):
        return self.stream.handle if self.stream else None

    @staticmethod
    def from_host(a: np.ndarray, dtype=None, stream: Stream | None = None) -> "DeviceTensor":
        a = np.ascontiguousarray(a, dtype=dtype or a.dtype)
        t = DeviceTensor(a.shape, a.dtype, stream)
        if t.nbytes:
            call("pcd_memcpy", t.ptr, a.ctypes.data, t.nbytes, MEMCPY["h2d"])
        return t

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            if self.stream:
                self.stream.synchronize()
            call("pcd_memcpy", out.ctypes.data, self.ptr, self.nbytes, MEMCPY["d2h"])
        return out

    def free(self) -> None:
        if getattr(self, "ptr", None):
            call("pcd_free_async", self.ptr, self._s())
        self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class TensorOps:
    """Device tensor operations (TensorOps.cs:24-86)."""

    @staticmethod
    def mat_mul(a: DeviceTensor, b: DeviceTensor, trans_a: bool = False, trans_b: bool = False,
                beta: float = 0.0, out: DeviceTensor | None = None, stream: Stream | None = None) -> DeviceTensor:
        """Row-major C = op(A) op(B) + beta C with an fp32 C (MatMulDeviceEx
        semantics): fp32 operands, fp16 operands (float16 tensors,
        MatMulMixedDevice) or bf16 operands (uint16 tensors of bf16 bits,
        MatMulDeviceExBf16).  Both operands must have the same type."""
        if len(a.shape) != 2 or len(b.shape) != 2:
            raise ArgumentException("MatMul needs 2-D tensors")
        if a.dtype != b.dtype or a.dtype not in _GEMM_FN:
            raise ArgumentException(f"MatMul operands must share one of float32, float16 or uint16 (bf16); "
                                    f"got {a.dtype} and {b.dtype}")
        m, k = (a.shape[1], a.shape[0]) if trans_a else a.shape
        k2, n = (b.shape[1], b.shape[0]) if trans_b else b.shape
        if k != k2:
            raise ArgumentException(f"inner dimensions differ: {k} vs {k2}")
        if out is None:
            out = DeviceTensor((m, n), np.float32, stream)
        fn = _GEMM_FN[a.dtype]
        call(fn, a.ptr, b.ptr, out.ptr, m, k, n, int(trans_a), int(trans_b), float(beta),
             stream.handle if stream else None)
        if stream is None:
            call("pcd_device_synchronize")
        return out

    @staticmethod
    def mat_mul_batched(a: DeviceTensor, b: DeviceTensor, out: DeviceTensor | None = None,
                        stream: Stream | None = None) -> DeviceTensor:
        """Strided batched product of [batch x m x k] and [batch x k x n] tensors
        into an fp32 [batch x m x n] (MatMulBatchedDevice, CudaGemmProvider.cs:130-141;
        16-bit operands as in mat_mul)."""
        if len(a.shape) != 3 or len(b.shape) != 3 or a.shape[0] != b.shape[0]:
            raise ArgumentException("batched MatMul needs [batch x m x k] and [batch x k x n] tensors")
        if a.dtype != b.dtype or a.dtype not in _GEMM_FN:
            raise ArgumentException(f"MatMul operands must share one of float32, float16 or uint16 (bf16); "
                                    f"got {a.dtype} and {b.dtype}")
        batch, m, k = a.shape
        _, k2, n = b.shape
        if k != k2:
            raise ArgumentException(f"inner dimensions differ: {k} vs {k2}")
        if out is None:
            out = DeviceTensor((batch, m, n), np.float32, stream)
        elif out.shape != (batch, m, n) or out.dtype != np.float32:
            raise ArgumentException("out must be an fp32 [batch x m x n] tensor")
        call(_GEMM_FN[a.dtype] + "_batched", a.ptr, b.ptr, out.ptr, batch, m, k, n, stream.handle if stream else None)
        if stream is None:
            call("pcd_device_synchronize")
        return out

    @staticmethod
    def copy_to(src: DeviceTensor, dst: DeviceTensor, stream: Stream | None = None) -> None:
        if src.nbytes != dst.nbytes:
            raise ArgumentException("size mismatch")
        call("pcd_memcpy_async", dst.ptr, src.ptr, src.nbytes, MEMCPY["d2d"], stream.handle if stream else None)

    @staticmethod
    def synchronize(stream: Stream | None = None) -> None:
        if stream:
            stream.synchronize()
        else:
            call("pcd_device_synchronize")
