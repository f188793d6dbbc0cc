"""Adaptive minimum-energy classification on the GPU (pcd_pc_classify_adaptive),
against the oracle's Network.PredictAdaptive (Network.cs:803-907) and the
reference's own adaptive-inference properties (AdaptiveInferenceTests.cs).

Bars: per candidate, the steps it ran equal the oracle's exactly (the relative
exit rule is decided on the same fp32 energies); energies within 1e-4 (fp32)
or 2e-3 (16-bit operands against the oracle with the same rounding); classes,
winner energies and steps used follow from those.
"""
import numpy as np
import pytest

from tests.netgen import make_inputs, make_net, max_rel

pytestmark = pytest.mark.gpu

ACT_ID = {"linear": 0, "tanh": 1, "relu": 2, "sigmoid": 3, "gelu": 4}


def _model(sizes, act, eta, W, b, P, ffg=False, dtype="f32"):
    from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel
    snap = GenerativeSnapshot(sizes, ACT_ID[act], eta, 0.0, ffg, W, b, list(P))
    return PcDeviceModel(snap, dtype)


def _check(got, want, tol, tag):
    ce, cs, bc, be, su = got
    rce, rcs, rbc, rbe, rsu = want
    print(f"{tag}: energies {max_rel(ce, rce):.2e}, steps equal {np.array_equal(cs, rcs)}, "
          f"exits {int(np.sum(rcs < rcs.max()))} of {rcs.size}", flush=True)
    assert np.array_equal(cs, rcs), (cs, rcs)
    assert max_rel(ce, rce) < tol and max_rel(be, rbe) < tol
    assert np.array_equal(su, rsu)
    # the class: the first minimum of the device's own energies, and the
    # oracle's wherever the two best candidates are apart by more than the bar
    assert np.array_equal(bc, np.argmin(ce, axis=1))
    srt = np.sort(rce, axis=1)
    clear = (srt[:, 1] - srt[:, 0]) > 4 * tol * (1 + srt[:, 0])
    assert np.array_equal(bc[clear], rbc[clear])
    assert np.array_equal(be, ce[np.arange(len(bc)), bc])
    assert np.array_equal(su, cs.sum(axis=1) + cs[np.arange(len(bc)), bc])


@pytest.mark.parametrize("act,ffg", [("tanh", False), ("gelu", True), ("sigmoid", False), ("relu", False)])
def test_classify_adaptive_fp32_matches_oracle(oracle, act, ffg):
    sizes = [12, 20, 9, 4]
    W, b, P = make_net(sizes, seed=51, bias_scale=0.2)
    x = make_inputs(5, 12, seed=52, dist="uniform01")
    m = _model(sizes, act, 0.1, W, b, P, ffg)
    try:
        for eps in (3e-2, 1e-2, 1e-3):
            got = m.classify_adaptive(x, 40, eps)
            want = oracle.classify_adaptive(sizes, act, 0.1, W, b, P, x, 40, eps, ffg=ffg)
            _check(got, want, 1e-4, f"adaptive/{act}/ffg{int(ffg)}/eps{eps:g}")
            assert np.any(got[1] < 40), "no candidate left early"
    finally:
        m.close()


@pytest.mark.parametrize("tile", [0, 32, 64, 128])
def test_classify_adaptive_c1_network(oracle, tile):
    # c1's network (784-256-256-10 tanh) with a batch of 24 samples: 240
    # one-row candidates, each with its own exit step
    sizes = [784, 256, 256, 10]
    W, b, P = make_net(sizes, seed=3)
    x = make_inputs(24, 784, seed=4, dist="uniform01")
    m = _model(sizes, "tanh", 0.1, W, b, P)
    try:
        if tile:
            m.set_option("tile", tile)
        got = m.classify_adaptive(x, 30, 2e-3)
        want = oracle.classify_adaptive(sizes, "tanh", 0.1, W, b, P, x, 30, 2e-3)
        _check(got, want, 1e-4, f"adaptive/c1/tile{tile}")
        assert np.any(got[1] < 30) and len(np.unique(got[1])) > 1   # candidates leave at different steps
    finally:
        m.close()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_classify_adaptive_16bit_operands(oracle, dtype):
    # With 16-bit operands the device's and the oracle's energies agree to a few
    # 1e-4 on this network (fp32 sums of the same rounded products, in another
    # order, and states rounded again every step), so a candidate whose
    # relative improvement lands that close to epsilon may stop one step apart.  Every candidate must either stop where the oracle
    # does, with its energy within 2e-3, or, one step apart, stop where the
    # oracle's own criterion is within that noise of epsilon, with the energy of
    # the oracle's trajectory at the device's step.
    sizes = [64, 128, 96, 6]
    W, b, P = make_net(sizes, seed=71, bias_scale=0.1)
    x = make_inputs(9, 64, seed=72, dist="uniform01")
    T, eps, C = 25, 1e-2, 6
    m = _model(sizes, "tanh", 0.1, W, b, P, dtype=dtype)
    try:
        ce, cs, bc, be, su = m.classify_adaptive(x, T, eps)
    finally:
        m.close()
    rce, rcs, rbc, rbe, rsu = oracle.classify_adaptive(sizes, "tanh", 0.1, W, b, P, x, T, eps, round_mode=dtype)
    same = cs == rcs
    print(f"adaptive/{dtype}: {int(same.sum())} of {same.size} candidates stop where the oracle does; energies "
          f"there {max_rel(ce[same], rce[same]):.2e}", flush=True)
    assert same.mean() >= 0.9
    err = max_rel(ce[same], rce[same])
    assert err < 2e-3
    # the improvement ratio (prev - E) / prev of two energies each off by err
    # is off by about 2 err: the noise an exit decision can fall within
    noise = 3 * err + 1e-5
    for i, c in np.argwhere(~same):
        top = np.zeros((1, C), np.float32)
        top[0, c] = 1.0
        _, tr = oracle.clamped_relax(sizes, "tanh", 0.1, W, b, P, x[i:i + 1], top, T, round_mode=dtype)
        tr = tr[:, 0].astype(np.float64)
        k, kr = int(cs[i, c]), int(rcs[i, c])
        j = min(k, kr)   # the earlier exit: the improvement of step j over step j - 1
        margin = (tr[j - 2] - tr[j - 1]) / max(tr[j - 2], 1e-12) - eps
        print(f"  sample {i} class {c}: device {k} steps, oracle {kr}; oracle criterion margin {margin:.1e}",
              flush=True)
        assert abs(k - kr) == 1 and abs(margin) < noise
        assert max_rel(ce[i, c], tr[k - 1]) < 2e-3
    # the outputs follow from the candidates as the reference composes them
    assert np.array_equal(bc, np.argmin(ce, axis=1))
    assert np.array_equal(be, ce[np.arange(len(bc)), bc])
    assert np.array_equal(su, cs.sum(axis=1) + cs[np.arange(len(bc)), bc])


def test_epsilon_zero_is_classify(oracle):
    # AdaptiveInferenceTests.cs:74-95: epsilon = 0 never exits, so the result is
    # the fixed-step classification, with stepsUsed = maxSteps * (C + 1)
    sizes = [40, 64, 32, 8]
    W, b, P = make_net(sizes, seed=81, bias_scale=0.1)
    x = make_inputs(20, 40, seed=82, dist="uniform01")
    m = _model(sizes, "tanh", 0.1, W, b, P)
    try:
        ce, cls, be = m.classify(x, 15)
        ace, acs, acls, abe, asu = m.classify_adaptive(x, 15, 0.0)
        print(f"eps 0 vs classify: energies {max_rel(ace, ce):.2e}", flush=True)
        assert np.array_equal(acls, cls)
        assert max_rel(ace, ce) < 1e-6 and max_rel(abe, be) < 1e-6
        assert np.all(acs == 15) and np.all(asu == 15 * (8 + 1))
    finally:
        m.close()


def test_trained_two_patterns_adaptive(oracle):
    # AdaptiveInferenceTests.cs:116-131: after TrainTwoPatterns a generous budget
    # (200) and epsilon 1e-3 classify both patterns, with finite non-negative
    # energies and fewer than 200 * (2 + 1) steps; and the effort presets run
    from predicitivecoding_amd import EffortLevel
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    a = np.array([[1, 0, 0, 0]], np.float32)
    bb = np.array([[0, 0, 0, 1]], np.float32)
    for _ in range(40):
        for x, y in ((a, [[1, 0]]), (bb, [[0, 1]])):
            W, b, _ = oracle.learn(sizes, "tanh", 0.1, W, b, P, x, np.array(y, np.float32), 30, 0.01)
    W = [np.ascontiguousarray(w, np.float32) for w in W]
    b = [np.ascontiguousarray(v, np.float32) for v in b]
    x = np.concatenate([a, bb])
    m = _model(sizes, "tanh", 0.1, W, b, P)
    try:
        _, cs, cls, be, su = m.classify_adaptive(x, 200, 1e-3)
        want = oracle.classify_adaptive(sizes, "tanh", 0.1, W, b, P, x, 200, 1e-3)
        _check((_, cs, cls, be, su), want, 1e-4, "adaptive/two patterns")
        assert list(cls) == [0, 1]
        assert np.all(np.isfinite(be)) and np.all(be >= 0)
        assert np.all(su < 200 * 3)
        spent = []
        for level in (EffortLevel.Low, EffortLevel.Medium, EffortLevel.High):
            c, e, u = m.predict_adaptive(x, level)
            assert list(c) == [0, 1] and np.all(np.isfinite(e))
            spent.append(int(u.sum()))
        assert spent[0] <= spent[1] <= spent[2]
    finally:
        m.close()


def test_classify_adaptive_graph_and_eager_agree_bit_for_bit():
    sizes = [40, 64, 32, 8]
    W, b, P = make_net(sizes, seed=91, bias_scale=0.1)
    xs = [make_inputs(20, 40, seed=92 + k, dist="uniform01") for k in range(2)]
    out = {}
    for graph in (1, 0):
        m = _model(sizes, "tanh", 0.1, W, b, P)
        try:
            m.set_option("use_graph", graph)
            # the same call shape twice: the second replays the cached graph with new inputs
            out[graph] = [m.classify_adaptive(x, 20, 1e-2) for x in xs]
        finally:
            m.close()
    for g, e in zip(out[1], out[0]):
        for a, c in zip(g, e):
            assert np.array_equal(a, c)
    assert not np.array_equal(out[1][0][0], out[1][1][0])


def test_classify_adaptive_argument_errors():
    from predicitivecoding_amd import ArgumentException, ArgumentOutOfRangeException, DeviceException
    from predicitivecoding_amd._native import lib
    sizes = [6, 10, 4]
    W, b, P = make_net(sizes, seed=1)
    m = _model(sizes, "tanh", 0.1, W, b, P)
    try:
        with pytest.raises(ArgumentOutOfRangeException):
            m.classify_adaptive(np.zeros((2, 6), np.float32), 0, 1e-3)
        with pytest.raises(ArgumentException):
            m.classify_adaptive(np.zeros((0, 6), np.float32), 10, 1e-3)
        x = np.zeros((2, 6), np.float32)
        assert lib().pcd_pc_classify_adaptive(m.handle, x.ctypes.data, 2, 10, 1e-3, None, None, None, None, None,
                                              None) == 4
        with pytest.raises(DeviceException):
            m.classify_adaptive_device(None, 2, 10, 1e-3, None, None, None, None, None)
    finally:
        m.close()
