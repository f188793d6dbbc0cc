"""MI355X-native batched predictive-coding relaxation (libpcdevice_hip).

Drop-in host mirror of the reference's PredictiveCoding.Device path:
BatchedPcForward.InferGetTopBatch, the GenerativeSnapshot handoff, the device
runtime (Device, DeviceTensor, TensorOps, streams) and the GEMM provider slot,
all computing through the hand-written gfx950 kernels in csrc/.
"""
from .batched_pc_forward import BatchedPcForward, PcDeviceModel
from .device import Device, DeviceKind, DeviceRuntime, DeviceTensor, Event, Stream, TensorOps
from .effort import EffortLevel, EffortPresets
from .errors import (ArgumentException, ArgumentNullException, ArgumentOutOfRangeException, DeviceException,
                     DeviceStatus, NotSupportedException)
from .gemm import Gemm, HipGemmProvider, IGemmProvider
from .registry import DeviceRegistry
from .snapshot import ActivationType, GenerativeSnapshot

__all__ = [
    "ActivationType", "ArgumentException", "ArgumentNullException", "ArgumentOutOfRangeException",
    "BatchedPcForward", "Device", "DeviceException", "DeviceRegistry", "DeviceKind", "DeviceRuntime", "DeviceStatus",
    "DeviceTensor", "EffortLevel", "EffortPresets", "Event", "Gemm", "GenerativeSnapshot", "HipGemmProvider", "IGemmProvider",
    "NotSupportedException", "PcDeviceModel", "Stream", "TensorOps",
]
