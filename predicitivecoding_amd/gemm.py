"""The pluggable GEMM boundary with an MI355X provider.

IGemmProvider mirrors PredictiveCoding.LLM/Infrastructure/Gemm.cs:17-27
(row-major C[m,n] = A[m,k] B[k,n]; MatMulMixed rounds both operands to 16
bits and accumulates in fp32).  HipGemmProvider runs both on the hand-written
gfx950 kernels through pcd_gemm_f32 / pcd_gemm_f16 (the role
CudaGemmProvider.MatMul / MatMulMixed play, CudaGemmProvider.cs:30-59,150-182).
"""
from __future__ import annotations

import numpy as np

from ._native import call
from .device import DeviceTensor
from .errors import ArgumentException


class IGemmProvider:
    def mat_mul(self, a, m: int, k: int, b, n: int) -> np.ndarray:
        raise NotImplementedError

    def mat_mul_mixed(self, a, m: int, k: int, b, n: int) -> np.ndarray:
        return self.mat_mul(a, m, k, b, n)


def _check(a, m, k, b, n):
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    b = np.ascontiguousarray(b, dtype=np.float32).ravel()
    if a.size != m * k:
        raise ArgumentException("A has wrong length.")
    if b.size != k * n:
        raise ArgumentException("B has wrong length.")
    return a, b


class HipGemmProvider(IGemmProvider):
    """The GPU provider on one device (CudaGemmProvider(deviceId), CudaGemmProvider.cs:19-28)."""

    def __init__(self, device_id: int = 0):
        self.device_id = int(device_id)

    def _device(self):
        call("pcd_set_device", self.device_id)

    def mat_mul(self, a, m, k, b, n):
        a, b = _check(a, m, k, b, n)
        self._device()
        with DeviceTensor.from_host(a) as da, DeviceTensor.from_host(b) as db, DeviceTensor((m, n)) as dc:
            call("pcd_gemm_f32", da.ptr, db.ptr, dc.ptr, m, k, n, 0, 0, 0.0, None)
            return dc.to_host()

    def mat_mul_mixed(self, a, m, k, b, n):
        a, b = _check(a, m, k, b, n)
        self._device()
        ah = a.astype(np.float16).view(np.uint16)
        bh = b.astype(np.float16).view(np.uint16)
        with DeviceTensor.from_host(ah) as da, DeviceTensor.from_host(bh) as db, DeviceTensor((m, n)) as dc:
            call("pcd_gemm_f16", da.ptr, db.ptr, dc.ptr, m, k, n, 0, 0, 0.0, None)
            return dc.to_host()

    def mat_mul_batched_device(self, dA: int, dB: int, dC: int, batch: int, m: int, k: int, n: int,
                               stream=None) -> None:
        """MatMulBatchedDevice (CudaGemmProvider.cs:130-141): C_i = A_i B_i for
        i < batch on device pointers, items m*k, k*n and m*n floats apart;
        queued on `stream`."""
        self._device()
        call("pcd_gemm_f32_batched", dA, dB, dC, int(batch), int(m), int(k), int(n),
             stream.handle if stream else None)


class Gemm:
    """Process-wide provider slot (Gemm.cs:63-73)."""

    provider: IGemmProvider = HipGemmProvider()

    @staticmethod
    def mat_mul(a, m, k, b, n):
        _check(a, m, k, b, n)
        return Gemm.provider.mat_mul(a, m, k, b, n)
