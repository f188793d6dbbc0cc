"""Weight records loaded straight into device operands (pcd_pc_model_load_record)
against the record restatement and the CPU oracle."""
import numpy as np
import pytest

from oracle import records as rec
from oracle.pc_oracle import ACT
from tests.netgen import make_inputs, make_net, max_rel

pytestmark = pytest.mark.gpu


def _records(sizes, W, b, P, fmt):
    out = [rec.serialize(sizes[0], 0, float(P[0]))]
    for l in range(1, len(sizes)):
        out.append(rec.serialize(sizes[l], sizes[l - 1], float(P[l]), W[l - 1], b[l - 1], fmt=fmt))
    return out


@pytest.mark.parametrize("fmt", [rec.FLOAT32, rec.HALF, rec.BF16, rec.INT8])
@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_records_into_device_operands(oracle, fmt, dtype):
    from predicitivecoding_amd import PcDeviceModel
    sizes = [37, 70, 19, 6]
    W, b, _ = make_net(sizes, seed=31, bias_scale=0.2)
    P = np.array([1.0, 0.8, 1.2, 1.0], np.float32)
    recs = _records(sizes, W, b, P, fmt)
    m = PcDeviceModel.from_records(recs, ACT["tanh"], 0.1, dtype=dtype)
    try:
        gw, gb = m.get_weights()
        x = make_inputs(9, sizes[0], seed=32)
        top, _, en = m.relax(x, 8, want_energy=True)
    finally:
        m.close()
    loaded = [rec.deserialize(r)[4] for r in recs[1:]]
    for l in range(3):
        # the widened record value (a 16-bit model's fp32 masters), bit for bit
        assert np.array_equal(gw[l], loaded[l]), (fmt, dtype, l)
        assert np.array_equal(gb[l], b[l])
    rtop, _, ren = oracle.batched_relax(sizes, "tanh", 0.1, loaded, b, P, x, 8, round_mode={"f32": "none"}.get(dtype, dtype),
                                        want_energy=True)
    tol = 1e-4 if dtype == "f32" else 2e-3
    errs = dict(top=max_rel(top, rtop), energy=max_rel(en, ren))
    print(f"record {fmt} -> {dtype}", errs, flush=True)
    assert all(v < tol for v in errs.values()), errs


@pytest.mark.parametrize("fmt", [rec.BF16, rec.INT8])
def test_quantized_persist_survives_reopen_with_same_classes(oracle, fmt):
    # MixedSub16Tests.PersistQuantized_SurvivesReopen_WithTheSameClasses (:124-163):
    # train two patterns, persist the layers quantized, reopen, same classes.
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    a = np.array([[1, 0, 0, 0]], np.float32)
    bb = np.array([[0, 0, 0, 1]], np.float32)
    oh = lambda c: np.eye(2, dtype=np.float32)[[c]]
    for _ in range(40):
        W, b, _ = oracle.learn(sizes, "tanh", 0.1, W, b, P, a, oh(0), 30, 0.01)
        W, b, _ = oracle.learn(sizes, "tanh", 0.1, W, b, P, bb, oh(1), 30, 0.01)
    _, cls_full, _ = oracle.classify(sizes, "tanh", 0.1, W, b, P, np.concatenate([a, bb]), 20)
    from predicitivecoding_amd import PcDeviceModel
    m = PcDeviceModel.from_records(_records(sizes, W, b, P, fmt), ACT["tanh"], 0.1)
    try:
        _, cls, _ = m.classify(np.concatenate([a, bb]), 20)
    finally:
        m.close()
    assert list(cls_full) == [0, 1] and list(cls) == [0, 1]


def test_record_errors():
    from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel
    from predicitivecoding_amd.errors import DeviceException, DeviceStatus
    sizes = [5, 4, 3]
    W, b, P = make_net(sizes, seed=1)
    m = PcDeviceModel(GenerativeSnapshot(sizes, ACT["tanh"], 0.1, 0.0, False, W, b, list(P)), "f32")
    try:
        bad = rec.serialize(3, 4, 1.0, np.zeros((4, 3)), np.zeros(4))         # layer 1 is (4, 5)
        with pytest.raises(DeviceException) as ei:
            m.load_record(1, bad)
        assert ei.value.code == DeviceStatus.InvalidValue and "Layer size mismatch" in str(ei.value)
        diag = bytearray(rec.serialize(4, 5, 1.0, np.zeros((5, 4)), np.zeros(5)))
        diag[25] |= 1
        with pytest.raises(DeviceException) as ei:
            m.load_record(1, bytes(diag) + b"\x00" * 16)
        assert ei.value.code == DeviceStatus.NotSupported
        with pytest.raises(DeviceException) as ei:
            m.load_record(1, rec.serialize(4, 5, 1.0, np.zeros((5, 4)), np.zeros(5))[:-4])
        assert ei.value.code == DeviceStatus.InvalidValue
    finally:
        m.close()
