"""DeviceRegistry: installs and restores the process-wide GEMM provider slot.

Host mirror of PredictiveCoding.Device/DeviceRegistry.cs:15-66 over
Gemm.provider (Gemm.cs:63-73).  enable_rocm installs the MI355X provider;
this package has no CPU compute path of its own, so use_cpu installs the CPU
provider the host application registered (its CpuGemmProvider) and refuses
when there is none, and auto_select raises when neither a GPU nor a
registered CPU provider is there.  installed() swaps a provider in for a
block and restores the previous one (the reference's tests serialise around
the slot, LlmGemmRouteTests.cs:13).
"""
from __future__ import annotations

from contextlib import contextmanager

from .device import Device, DeviceRuntime
from .errors import DeviceException, DeviceStatus, NotSupportedException
from .gemm import Gemm, HipGemmProvider, IGemmProvider


class DeviceRegistry:
    cuda_enabled = False    # no CUDA backend in this build
    rocm_enabled = False
    _cpu_provider: IGemmProvider | None = None

    @staticmethod
    def default_device() -> Device:
        """DefaultDevice (DeviceRegistry.cs:21): the GPU when one is present."""
        return Device.rocm(0) if DeviceRuntime.available() else Device.cpu()

    @classmethod
    def enable_rocm(cls, device_id: int = 0) -> bool:
        """EnableRocm (DeviceRegistry.cs:44-50): installs the GPU provider;
        true if a real device is present (its calls raise otherwise)."""
        Gemm.provider = HipGemmProvider(device_id)
        cls.cuda_enabled = False
        cls.rocm_enabled = DeviceRuntime.available()
        return cls.rocm_enabled

    @classmethod
    def enable_cuda(cls, device_id: int = 0) -> bool:
        raise NotSupportedException("this build has no CUDA backend; enable_rocm installs the MI355X provider")

    @classmethod
    def register_cpu_provider(cls, provider: IGemmProvider | None) -> None:
        """The host application's CPU provider, which use_cpu and auto_select install."""
        cls._cpu_provider = provider

    @classmethod
    def use_cpu(cls) -> None:
        """UseCpu (DeviceRegistry.cs:53-58) with the registered CPU provider."""
        if cls._cpu_provider is None:
            raise NotSupportedException("no CPU GEMM provider registered (this package computes only on the GPU)")
        Gemm.provider = cls._cpu_provider
        cls.cuda_enabled = False
        cls.rocm_enabled = False

    @classmethod
    def auto_select(cls) -> Device:
        """AutoSelect (DeviceRegistry.cs:61-66): the GPU when present, else the
        registered CPU provider."""
        if DeviceRuntime.available():
            cls.enable_rocm()
        elif cls._cpu_provider is not None:
            cls.use_cpu()
        else:
            raise DeviceException(DeviceStatus.NoDevice, "DeviceRegistry.auto_select",
                                  "no GPU and no CPU GEMM provider registered")
        return cls.default_device()

    @classmethod
    @contextmanager
    def installed(cls, provider: IGemmProvider):
        """Gemm.provider = provider for the block, then the previous provider
        and flags again."""
        saved = (Gemm.provider, cls.cuda_enabled, cls.rocm_enabled)
        Gemm.provider = provider
        try:
            yield provider
        finally:
            Gemm.provider, cls.cuda_enabled, cls.rocm_enabled = saved
