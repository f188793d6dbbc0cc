"""The C ABI library loads, exports every declared symbol, and rejects bad
arguments with the reference's status codes before touching a GPU."""
import ctypes

import numpy as np
import pytest

from predicitivecoding_amd import _native
from predicitivecoding_amd.errors import ArgumentException, DeviceException, DeviceStatus, NotSupportedException


def test_library_exports_every_declared_symbol():
    syms = _native.header_symbols()
    assert len(syms) >= 30
    L = _native.lib()
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    assert set(syms) == set(_native._SIGNATURES), set(syms) ^ set(_native._SIGNATURES)


def test_header_is_plain_c_and_the_c_client_links(tmp_path):
    # include/pcdevice.h is the whole boundary for a C caller: the C99 client
    # compiles with -pedantic and links against the library and the oracle
    import os
    import subprocess
    here = os.path.dirname(os.path.abspath(__file__))
    src = os.path.join(here, "c_client", "relax_client.c")
    root = os.path.dirname(here)
    out = str(tmp_path / "relax_client")
    res = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I" + os.path.join(root, "include"),
                          src, "-o", out, "-L" + os.path.join(root, "predicitivecoding_amd"), "-lpcdevice_hip",
                          "-L" + os.path.join(root, "oracle"), "-lpcoracle", "-lm"], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr


def test_status_codes_match_reference_enum():
    # Interop/CudaStatus.cs:7-19
    want = {"Success": 0, "NotInitialized": 1, "NoDevice": 2, "OutOfMemory": 3, "InvalidValue": 4,
            "NotSupported": 8, "Unknown": 100}
    for k, v in want.items():
        assert DeviceStatus[k] == v
    text = open(_native.HEADER).read()
    for name, v in [("PCD_SUCCESS", 0), ("PCD_NO_DEVICE", 2), ("PCD_INVALID_VALUE", 4), ("PCD_NOT_SUPPORTED", 8)]:
        assert f"{name} = {v}" in text


def test_version_and_last_error():
    v = ctypes.c_int()
    assert _native.lib().pcd_version(ctypes.byref(v)) == 0 and v.value >= 100
    assert _native.lib().pcd_pc_relax(None, None, 1, 1, None, None, None, None) == DeviceStatus.NotInitialized
    assert "null model" in _native.last_error()


def test_argument_errors_without_gpu():
    L = _native.lib()
    assert L.pcd_gemm_f32(None, None, None, 2, 2, 2, 0, 0, 0.0, None) == DeviceStatus.InvalidValue
    out = ctypes.c_void_p()
    sizes = (ctypes.c_int * 1)(4)
    assert L.pcd_pc_model_create(sizes, 1, 1, 0.1, 0.0, 0, None, None, None, 0, ctypes.byref(out)) == \
        DeviceStatus.InvalidValue
    sizes2 = (ctypes.c_int * 2)(4, 3)
    w = (ctypes.c_void_p * 1)(None)
    prec = (ctypes.c_float * 2)(1.0, 1.0)
    # unknown activation, unknown dtype, non-positive precision
    assert L.pcd_pc_model_create(sizes2, 2, 9, 0.1, 0.0, 0, w, w, prec, 0, ctypes.byref(out)) == DeviceStatus.InvalidValue
    assert L.pcd_pc_model_create(sizes2, 2, 1, 0.1, 0.0, 0, w, w, prec, 7, ctypes.byref(out)) == DeviceStatus.InvalidValue
    bad = (ctypes.c_float * 2)(1.0, 0.0)
    assert L.pcd_pc_model_create(sizes2, 2, 1, 0.1, 0.0, 0, w, w, bad, 0, ctypes.byref(out)) == DeviceStatus.InvalidValue
    assert L.pcd_free_async(ctypes.c_void_p(12345), None) == DeviceStatus.InvalidValue
    assert L.pcd_memcpy(None, None, 4, 9) == DeviceStatus.InvalidValue
    with pytest.raises(DeviceException) as ei:
        _native.call("pcd_memcpy", None, None, 4, 1)
    assert ei.value.code == DeviceStatus.InvalidValue


def test_host_mirror_argument_validation():
    # BatchedPcForwardTests.cs:120-132 and :113-118, raised before any device call
    from predicitivecoding_amd import (ArgumentOutOfRangeException, BatchedPcForward, GenerativeSnapshot)
    sizes = [6, 10, 4]
    W = [np.zeros((6, 10), np.float32), np.zeros((10, 4), np.float32)]
    b = [np.zeros(6, np.float32), np.zeros(10, np.float32)]
    snap = GenerativeSnapshot(sizes, 1, 0.1, 0.0, False, W, b, [1.0, 1.0, 1.0])
    with pytest.raises(ArgumentException):
        BatchedPcForward.infer_get_top_batch(snap, [], 5)
    with pytest.raises(ArgumentOutOfRangeException):
        BatchedPcForward.infer_get_top_batch(snap, [np.zeros(6)] * 2, 0)
    with pytest.raises(ArgumentException):
        BatchedPcForward.infer_get_top_batch(snap, [np.zeros(5)] * 2, 5)
    with pytest.raises(NotSupportedException):
        GenerativeSnapshot(sizes, 1, 0.1, 0.0, False, W, b, [1.0, np.ones(10), 1.0])
    with pytest.raises(NotSupportedException):
        GenerativeSnapshot(sizes, 1, 0.1, 0.0, False, W, b, [1.0, 1.0, 1.0], prior_mean=np.zeros(4))
    with pytest.raises(ArgumentException):
        GenerativeSnapshot(sizes, 1, 0.1, 0.0, False, [W[1], W[0]], b, [1.0, 1.0, 1.0])


def test_no_device_reported_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    n = ctypes.c_int(-1)
    assert _native.lib().pcd_get_device_count(ctypes.byref(n)) == DeviceStatus.NoDevice
    assert n.value == 0


def test_clamped_classify_learn_argument_errors_without_gpu():
    # null model handle first (NotInitialized), before any device work
    L = _native.lib()
    assert L.pcd_pc_relax_clamped(None, None, None, 1, 1, None, None, None) == DeviceStatus.NotInitialized
    assert L.pcd_pc_classify(None, None, 1, 1, None, None, None, None) == DeviceStatus.NotInitialized
    assert L.pcd_pc_learn(None, None, None, 1, 1, 0.01, 0.0, None, None) == DeviceStatus.NotInitialized
    assert L.pcd_pc_model_get_weights(None, 1, None, None) == DeviceStatus.NotInitialized


def test_snapshot_is_an_immutable_copy():
    # The drop-in uploads a snapshot's weights once and reuses the device copy
    # (BatchedPcForward.cs:62-64 re-reads them per call instead): the snapshot
    # therefore owns read-only copies.  Editing the caller's arrays afterwards
    # does not reach it, editing through it is refused, and so is replacing a
    # field.
    from predicitivecoding_amd import GenerativeSnapshot
    sizes = [6, 10, 4]
    W = [np.ones((6, 10), np.float32), np.ones((10, 4), np.float32)]
    b = [np.zeros(6, np.float32), np.zeros(10, np.float32)]
    snap = GenerativeSnapshot(sizes, 1, 0.1, 0.0, False, W, b, [1.0, 1.0, 1.0])
    assert snap.weights[0] is not W[0] and not np.shares_memory(snap.weights[0], W[0])
    W[0][0, 0] = 5.0
    b[1][3] = 2.0
    assert snap.weights[0][0, 0] == 1.0 and snap.biases[1][3] == 0.0
    with pytest.raises(ValueError):
        snap.weights[0][0, 0] = 5.0
    with pytest.raises(ValueError):
        snap.biases[0][0] = 1.0
    with pytest.raises(NotSupportedException):
        snap.weights = [W[0] * 2, W[1]]
    with pytest.raises(NotSupportedException):
        snap.state_learning_rate = 0.5
    with pytest.raises(TypeError):
        snap.weights[0] = W[0]          # a tuple: the layer list cannot be edited either
