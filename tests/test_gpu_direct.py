"""The direct-weight tile: batches of up to 64 rows of a 16-bit model whose
weight operand goes from a fragment-major copy straight into registers.
Networks with at least one such tile per CU in their error phase (c5's at
64 rows) take it by themselves; the option direct = 2 forces it on small
ones, so that odd shapes, the epilogues, FFG, learning (which rewrites the
copies) and the ragged and allocation-free calls are all covered.  Held to the
16-bit tiles' bounds: 2e-3 against the oracle with the same operand rounding,
2e-2 against fp32.
"""
import numpy as np
import pytest

from tests.gpu_util import build_case, run_gpu, run_oracle
from tests.netgen import make_inputs, max_rel

pytestmark = pytest.mark.gpu

CASES = [
    # sizes, activation, ffg, act_reg, batch, dtype, seed
    ([96, 130, 64, 16], "gelu", False, 0.0, 40, "bf16", 5),
    ([96, 130, 64, 16], "tanh", False, 0.0, 64, "f16", 6),
    ([784, 256, 256, 10], "tanh", True, 0.0, 64, "bf16", 7),
    ([100, 37, 300, 64, 5], "tanh", False, 0.05, 1, "bf16", 8),
    ([513, 700, 129], "sigmoid", True, 0.0, 17, "f16", 9),
    ([300, 520, 260, 70], "linear", False, 0.0, 33, "bf16", 10),
    ([64, 2048, 1024, 32], "relu", False, 0.0, 64, "bf16", 11),
]


def _report(name, **errs):
    print(name + ": " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_direct_tile_against_oracle(oracle, case):
    sizes, act, ffg, lam, B, dtype, seed = CASES[case]
    print(f"direct case {case}: {sizes} {act} ffg {ffg} act_reg {lam} batch {B} {dtype}", flush=True)
    snap, W, b, P, x = build_case(sizes, act, 0.05, act_reg=lam, ffg=ffg, batch=B, seed=seed, init="fanin",
                                  bias_scale=0.1)
    top, st, en = run_gpu(snap, x, 10, dtype=dtype, states=True, energy=True, options={"direct": 2})
    rtop, rst, ren = run_oracle(oracle, snap, W, b, P, x, 10, dtype=dtype, states=True, energy=True)
    ftop, _, fen = run_oracle(oracle, snap, W, b, P, x, 10, dtype="f32", energy=True)
    errs = dict(top=max_rel(top, rtop), energy=max_rel(en, ren),
                states=max(max_rel(a, r) for a, r in zip(st, rst)),
                top_vs_f32=max_rel(top, ftop), energy_vs_f32=max_rel(en, fen))
    _report(f"direct {case}", **errs)
    assert errs["top"] < 2e-3 and errs["energy"] < 2e-3 and errs["states"] < 2e-3, errs
    assert errs["top_vs_f32"] < 2e-2 and errs["energy_vs_f32"] < 2e-2, errs


def test_direct_tile_on_c5_network_at_64_rows(oracle):
    # BASELINE configs[4]'s network (12 x 8192 GELU bf16, eta 0.02) at a batch of 64: the library
    # chooses the direct-weight tile itself (the option at 0 gives the 64 x 64 tile, whose sums run
    # in another order, so the two differ in the last bits); a row subset against the oracle.
    # T = 14: from zero states the input reaches the top layer after 11 steps.
    sizes, B, T = [8192] * 12, 64, 14
    snap, W, b, P, x = build_case(sizes, "gelu", 0.02, batch=B, seed=31, init="fanin")
    top, _, en = run_gpu(snap, x, T, dtype="bf16", energy=True)
    top0, _, en0 = run_gpu(snap, x, T, dtype="bf16", energy=True, options={"direct": 0})
    assert np.abs(top).max() > 0
    assert not np.array_equal(top, top0), "the default call did not take the direct-weight tile"
    rows = np.array([0, 9, 30, 63])
    rtop, _, ren = run_oracle(oracle, snap, W, b, P, x[rows], T, dtype="bf16", energy=True)
    ftop, _, fen = run_oracle(oracle, snap, W, b, P, x[rows], T, dtype="f32", energy=True)
    errs = dict(top=max_rel(top[rows], rtop), energy=max_rel(en[:, rows], ren),
                top_vs_f32=max_rel(top[rows], ftop), energy_vs_f32=max_rel(en[:, rows], fen),
                vs_64x64=max_rel(top, top0))
    _report("c5 network, 64 rows", **errs)
    assert errs["top"] < 2e-3 and errs["energy"] < 2e-3, errs
    assert errs["top_vs_f32"] < 2e-2 and errs["energy_vs_f32"] < 2e-2 and errs["vs_64x64"] < 2e-3, errs


@pytest.mark.parametrize("batch", [9, 64])
def test_direct_tile_after_learning(oracle, batch):
    # the learning step rewrites the operand copies (one-launch update at these batches), and the
    # fragment-major copies with them: the settling after it sees the new weights
    from predicitivecoding_amd import PcDeviceModel
    sizes = [37, 70, 19, 6]
    snap, W, b, P, x = build_case(sizes, "gelu", 0.1, batch=batch, bias_scale=0.1, seed=17)
    y = np.eye(6, dtype=np.float32)[np.arange(batch) % 6]
    m = PcDeviceModel(snap, "bf16")
    try:
        m.set_option("direct", 2)
        en = m.learn(x, y, 8, 0.05)
        top, _, en2 = m.relax(x, 6, want_energy=True)
    finally:
        m.close()
    rw, rb, ren = oracle.learn(sizes, "gelu", 0.1, W, b, P, x, y, 8, 0.05, round_mode="bf16")
    rtop, _, ren2 = oracle.batched_relax(sizes, "gelu", 0.1, rw, rb, P, x, 6, round_mode="bf16", want_energy=True)
    errs = dict(energy=max_rel(en, ren), top_after=max_rel(top, rtop), energy_after=max_rel(en2, ren2))
    _report(f"direct learn {batch}", **errs)
    assert all(v < 2e-3 for v in errs.values()), errs


def test_direct_tile_ragged(oracle):
    from predicitivecoding_amd import PcDeviceModel
    sizes = [40, 64, 32, 8]
    snap, W, b, P, _ = build_case(sizes, "tanh", 0.1, seed=17)
    rng = np.random.default_rng(3)
    counts = [1, 5, 17, 2, 9, 3, 20]
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    x = (rng.standard_normal((offs[-1], sizes[0])) * 0.3).astype(np.float32)
    steps = rng.integers(3, 30, len(counts)).astype(np.int32)
    m = PcDeviceModel(snap, "bf16")
    try:
        m.set_option("direct", 2)
        used, fe, top = m.relax_ragged(x, offs, steps, "none")
    finally:
        m.close()
    rused, rfe, rtop = oracle.ragged_relax(sizes, "tanh", 0.1, W, b, P, x, offs, steps, "none", round_mode="bf16")
    errs = dict(top=max_rel(top, rtop), energy=max_rel(fe, rfe))
    _report("direct ragged", **errs)
    assert np.array_equal(used, steps) and np.array_equal(rused, steps)
    assert all(v < 2e-3 for v in errs.values()), errs


def test_direct_tile_noalloc_matches_relax():
    # the allocation-free call takes the same tile, so it matches pcd_pc_relax bit for bit
    from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel
    from tests.netgen import make_net
    from tests.test_zz_no_alloc import _run
    sizes = [256, 512, 64, 10]
    W, b, P = make_net(sizes, seed=3, bias_scale=0.1)
    m = PcDeviceModel(GenerativeSnapshot(sizes, 4, 0.05, 0.0, False, W, b, list(P)), "bf16")
    try:
        m.set_option("direct", 2)
        for B in (64, 23):
            x = make_inputs(B, sizes[0], seed=B)
            a = _run("pcd_pc_relax", m, x, 5)
            n = _run("pcd_pc_relax_noalloc", m, x, 5)
            for u, v in zip(a, n):
                assert np.array_equal(u, v)
    finally:
        m.close()


def test_direct_option_values():
    from predicitivecoding_amd import PcDeviceModel
    from predicitivecoding_amd.errors import DeviceException
    snap, *_ = build_case([32, 16, 8], "tanh", 0.1)
    m = PcDeviceModel(snap, "f32")
    try:
        m.set_option("direct", 0)
        m.set_option("direct", 1)
        for bad in (-1, 3):
            with pytest.raises(DeviceException):
                m.set_option("direct", bad)
        with pytest.raises(DeviceException):
            m.set_option("direct", 2)   # fp32 model
    finally:
        m.close()
