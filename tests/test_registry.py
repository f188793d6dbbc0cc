"""DeviceRegistry (DeviceRegistry.cs:15-66) over the Gemm.provider slot, on the
CPU: installing, restoring and selecting providers needs no GPU call."""
import numpy as np
import pytest

from predicitivecoding_amd import (DeviceException, DeviceRegistry, Gemm, HipGemmProvider, IGemmProvider,
                                   NotSupportedException)


class _HostProvider(IGemmProvider):
    """A stand-in for the host application's CPU provider (the test's own)."""

    def __init__(self):
        self.calls = 0

    def mat_mul(self, a, m, k, b, n):
        self.calls += 1
        return np.zeros((m, n), np.float32)


@pytest.fixture
def slot():
    saved = (Gemm.provider, DeviceRegistry.cuda_enabled, DeviceRegistry.rocm_enabled, DeviceRegistry._cpu_provider)
    yield
    Gemm.provider, DeviceRegistry.cuda_enabled, DeviceRegistry.rocm_enabled, DeviceRegistry._cpu_provider = saved


def test_enable_rocm_installs_the_gpu_provider(slot):
    DeviceRegistry.register_cpu_provider(None)
    present = DeviceRegistry.enable_rocm(0)
    assert isinstance(Gemm.provider, HipGemmProvider) and Gemm.provider.device_id == 0
    assert DeviceRegistry.rocm_enabled == present and not DeviceRegistry.cuda_enabled
    with pytest.raises(NotSupportedException):
        DeviceRegistry.enable_cuda()


def test_use_cpu_installs_the_registered_provider_or_refuses(slot):
    DeviceRegistry.register_cpu_provider(None)
    with pytest.raises(NotSupportedException):
        DeviceRegistry.use_cpu()
    host = _HostProvider()
    DeviceRegistry.register_cpu_provider(host)
    DeviceRegistry.enable_rocm()
    DeviceRegistry.use_cpu()
    assert Gemm.provider is host and not DeviceRegistry.rocm_enabled
    Gemm.mat_mul(np.ones(6, np.float32), 2, 3, np.ones(12, np.float32), 4)
    assert host.calls == 1


def test_installed_restores_the_previous_provider(slot):
    before = Gemm.provider
    host = _HostProvider()
    with DeviceRegistry.installed(host):
        assert Gemm.provider is host
    assert Gemm.provider is before
    with pytest.raises(RuntimeError):
        with DeviceRegistry.installed(host):
            raise RuntimeError("inside")
    assert Gemm.provider is before


def test_auto_select_without_a_gpu(slot):
    from predicitivecoding_amd import DeviceRuntime
    if DeviceRuntime.available():
        pytest.skip("a GPU is present: auto_select installs it (covered by the GPU tests)")
    DeviceRegistry.register_cpu_provider(None)
    with pytest.raises(DeviceException):
        DeviceRegistry.auto_select()
    host = _HostProvider()
    DeviceRegistry.register_cpu_provider(host)
    assert DeviceRegistry.auto_select().is_cpu and Gemm.provider is host
