"""Strided batched GEMM (pcd_gemm_{f32,bf16,f16}_batched; MatMulBatchedDevice,
CudaGemmProvider.cs:130-141) against float64, and the registry's GPU provider.

Bars: fp32 operands 1e-5 relative to the float64 product of the same values
(|a-b| <= tol (1 + |b|) scaled by sqrt(k)); 16-bit operands against the float64
product of the rounded operands at the same bar (the accumulation is fp32 in
both kernels, the rounding is the operands' only).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1, 1, 1), (3, 37, 53, 29), (5, 64, 64, 64), (2, 200, 130, 333), (37, 8, 16, 8), (4, 512, 256, 384),
          # many items: the tile is chosen from the item's own size (never larger
          # than it), with the item count deciding among the tiles that fit --
          # 64 x 64 for 512 small items, 128 x 128 (f32) and 256 x 256 (16-bit)
          # when the items are that large and numerous enough to fill the CUs
          (512, 64, 64, 64), (300, 128, 64, 128), (256, 256, 64, 256)]


def _round(x, dtype):
    import torch
    t = torch.from_numpy(x)
    if dtype == "bf16":
        r = t.to(torch.bfloat16)
        return r.float().numpy(), r.view(torch.int16).numpy().view(np.uint16)
    r = t.to(torch.float16)
    return r.float().numpy(), r.numpy()


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES)
def test_batched_gemm_against_float64(dtype, shape):
    from predicitivecoding_amd import DeviceTensor, TensorOps
    batch, m, k, n = shape
    rng = np.random.default_rng(batch * 1000 + m)
    A = rng.standard_normal((batch, m, k)).astype(np.float32)
    B = rng.standard_normal((batch, k, n)).astype(np.float32)
    if dtype == "f32":
        Av, Bv, Ad, Bd = A, B, A, B
    else:
        Av, Ad = _round(A, dtype)
        Bv, Bd = _round(B, dtype)
    want = np.einsum("bmk,bkn->bmn", Av.astype(np.float64), Bv.astype(np.float64))
    da, db = DeviceTensor.from_host(Ad), DeviceTensor.from_host(Bd)
    try:
        got = TensorOps.mat_mul_batched(da, db).to_host()
    finally:
        da.free()
        db.free()
    err = float(np.max(np.abs(got - want) / (1 + np.abs(want))))
    print(f"batched {dtype} {shape}: {err:.2e}", flush=True)
    assert got.shape == (batch, m, n)
    assert err < 1e-5 * np.sqrt(k)
    # every item is its own product (no item reads another's operands)
    for i in (0, batch - 1):
        assert np.allclose(got[i], Av[i].astype(np.float64) @ Bv[i].astype(np.float64), rtol=1e-4, atol=1e-4 * np.sqrt(k))


def test_provider_batched_device_and_registry_route():
    from predicitivecoding_amd import DeviceRegistry, DeviceTensor, Gemm, HipGemmProvider
    saved = Gemm.provider
    try:
        assert DeviceRegistry.enable_rocm(0) is True
        assert isinstance(Gemm.provider, HipGemmProvider) and DeviceRegistry.rocm_enabled
        assert not DeviceRegistry.default_device().is_cpu
        rng = np.random.default_rng(7)
        A = rng.standard_normal((6, 33, 47)).astype(np.float32)
        B = rng.standard_normal((6, 47, 21)).astype(np.float32)
        da, db, dc = DeviceTensor.from_host(A), DeviceTensor.from_host(B), DeviceTensor((6, 33, 21))
        try:
            Gemm.provider.mat_mul_batched_device(da.ptr, db.ptr, dc.ptr, 6, 33, 47, 21)
            got = dc.to_host()
        finally:
            for t in (da, db, dc):
                t.free()
        want = A.astype(np.float64) @ B.astype(np.float64)
        assert np.max(np.abs(got - want) / (1 + np.abs(want))) < 1e-5 * np.sqrt(47)
        # the slot routes the plain GEMM through the GPU provider (LlmDeviceTests.cs:41-55)
        c = Gemm.mat_mul(np.array([1, 2, 3, 4, 5, 6], np.float32), 2, 3,
                         np.array([7, 8, 9, 10, 11, 12], np.float32), 2)
        assert c.tolist() == [[58, 64], [139, 154]]
    finally:
        Gemm.provider = saved


def test_batched_gemm_argument_errors():
    from predicitivecoding_amd import ArgumentException, DeviceException, DeviceTensor, TensorOps
    from predicitivecoding_amd._native import call
    a = DeviceTensor.from_host(np.zeros((2, 3, 4), np.float32))
    b = DeviceTensor.from_host(np.zeros((2, 5, 6), np.float32))
    try:
        with pytest.raises(ArgumentException):
            TensorOps.mat_mul_batched(a, b)
        with pytest.raises(DeviceException):
            call("pcd_gemm_f32_batched", a.ptr, b.ptr, None, 2, 3, 4, 6, None)
        with pytest.raises(DeviceException):
            call("pcd_gemm_f32_batched", a.ptr, b.ptr, a.ptr, 0, 3, 4, 6, None)
    finally:
        a.free()
        b.free()
