"""The persistent settling (one cooperative launch for the whole step loop,
grid barriers between the phases; option `persistent`, off by default) on the
small fp32 configurations.

It runs the phase kernels' own work units on 64 x 64 tiles, so its results
must equal the per-phase launches' on the same tiles bit for bit (the
automatic choice for these networks without the persistent form is the
K-shared 32 x 32 tile, which sums K in another order); and the oracle's within
1e-4.  Its grid
barrier gives up after a bounded number of polls: forced from the host with a
spin limit of one poll, the call reports PCD_HIP_ERROR, every workgroup exits
normally, and the next call on the same model is correct again.
"""
import numpy as np
import pytest

from tests.gpu_util import build_case, run_oracle
from tests.netgen import max_rel

pytestmark = pytest.mark.gpu

CASES = [
    # sizes, act, eta, batch, steps, ffg
    ([784, 256, 256, 10], "tanh", 0.1, 64, 20, False),
    ([784, 256, 256, 10], "tanh", 0.1, 20, 7, False),
    ([96, 200, 130, 7], "gelu", 0.1, 5, 12, True),
    ([40, 64, 32, 8], "sigmoid", 0.1, 33, 9, False),
    ([300, 512, 512, 64, 16], "relu", 0.05, 64, 10, False),
]


def _relax(snap, x, steps, persistent, dtype="f32"):
    from predicitivecoding_amd import PcDeviceModel
    m = PcDeviceModel(snap, dtype)
    try:
        m.set_option("tile", 64)
        m.set_option("persistent", persistent)
        return m.relax(x, steps, want_states=True, want_energy=True)
    finally:
        m.close()


@pytest.mark.parametrize("case", range(len(CASES)))
def test_persistent_matches_phase_launches_and_oracle(oracle, case):
    sizes, act, eta, batch, steps, ffg = CASES[case]
    print(f"persistent case {case}: {sizes} {act} B={batch} T={steps} ffg={ffg}", flush=True)
    snap, W, b, P, x = build_case(sizes, act, eta, ffg=ffg, batch=batch, seed=40 + case, bias_scale=0.1)
    top1, st1, en1 = _relax(snap, x, steps, 1)
    top0, st0, en0 = _relax(snap, x, steps, 0)
    assert np.array_equal(top1, top0) and np.array_equal(en1, en0)
    assert all(np.array_equal(a, c) for a, c in zip(st1, st0))
    rtop, rst, ren = run_oracle(oracle, snap, W, b, P, x, steps, states=True, energy=True)
    err = max(max_rel(top1, rtop), max_rel(en1, ren), max(max_rel(a, c) for a, c in zip(st1, rst)))
    print(f"  bit-identical to the phase launches; vs oracle {err:.2e}", flush=True)
    assert err < 1e-4


def test_persistent_clamped_settling(oracle):
    from predicitivecoding_amd import PcDeviceModel
    sizes = [784, 256, 256, 10]
    snap, W, b, P, x = build_case(sizes, "tanh", 0.1, batch=64, seed=7)
    y = np.eye(10, dtype=np.float32)[np.arange(64) % 10]
    out = {}
    for persistent in (1, 0):
        m = PcDeviceModel(snap, "f32")
        try:
            m.set_option("tile", 64)
            m.set_option("persistent", persistent)
            out[persistent] = m.relax_clamped(x, y, 15, want_states=True)
        finally:
            m.close()
    (s1, e1), (s0, e0) = out[1], out[0]
    assert np.array_equal(e1, e0) and all(np.array_equal(a, c) for a, c in zip(s1, s0))
    _, ren = oracle.clamped_relax(sizes, "tanh", 0.1, W, b, P, x, y, 15)
    assert max_rel(e1, ren) < 1e-4


def test_persistent_barrier_gives_up_and_recovers(oracle):
    from predicitivecoding_amd import DeviceException, PcDeviceModel
    sizes = [784, 256, 256, 10]
    snap, W, b, P, x = build_case(sizes, "tanh", 0.1, batch=64, seed=9)
    m = PcDeviceModel(snap, "f32")
    try:
        m.set_option("persistent", 1)
        m.set_option("persist_spin", 1)
        with pytest.raises(DeviceException) as ei:
            m.relax(x, 20)
        assert ei.value.code == 5 and "gave up" in str(ei.value)
        # a give-up can leave a split tile's ranges half counted; the next
        # call, persistent or not, must still settle correctly
        m.set_option("persist_spin", 1 << 22)
        top, _, en = m.relax(x, 20, want_energy=True)
        with pytest.raises(DeviceException):
            m.set_option("persist_spin", 1)
            m.relax(x, 20)
        m.set_option("persist_spin", 1 << 22)
        m.set_option("persistent", 0)
        top0, _, en0 = m.relax(x, 20, want_energy=True)
    finally:
        m.close()
    rtop, _, ren = run_oracle(oracle, snap, W, b, P, x, 20, energy=True)
    assert max_rel(top, rtop) < 1e-4 and max_rel(en, ren) < 1e-4
    assert max_rel(top0, rtop) < 1e-4 and max_rel(en0, ren) < 1e-4


def test_persistent_grid_options():
    # any grid that is a multiple of 8 computes the same bits (the units do not
    # depend on which workgroup runs them; more than can be resident is
    # capped); other values are refused
    from predicitivecoding_amd import DeviceException, PcDeviceModel
    snap, W, b, P, x = build_case([784, 256, 256, 10], "tanh", 0.1, batch=64, seed=11)
    outs = []
    m = PcDeviceModel(snap, "f32")
    try:
        m.set_option("persistent", 1)
        for g in (0, 8, 64, 4096):
            m.set_option("persist_grid", g)
            outs.append(m.relax(x, 10, want_energy=True))
        with pytest.raises(DeviceException):
            m.set_option("persist_grid", 12)
    finally:
        m.close()
    for o in outs[1:]:
        assert np.array_equal(o[0], outs[0][0]) and np.array_equal(o[2], outs[0][2])
