"""GPU parity of the clamped-top settling, minimum-energy classification and
learning step against the CPU oracle, through the C ABI.

Bounds |a-b| <= tol*(1+|b|) as in BatchedPcForwardTests.cs:67:
  fp32 states / energies / weights          1e-4
  16-bit operands vs the same-rounding oracle 2e-3
The predicted class must equal the oracle's wherever the oracle's best and
second-best class energies differ by more than the energy tolerance (a closer
pair is a tie at fp32 accuracy; either class is then accepted).
"""
import numpy as np
import pytest

from oracle.pc_oracle import ACT
from predicitivecoding_amd.errors import ArgumentException
from tests.gpu_util import ROUND, build_case
from tests.netgen import make_inputs, make_net, max_rel

pytestmark = pytest.mark.gpu

ACT_NAME = {v: k for k, v in ACT.items()}


def _report(name, **errs):
    print(name, " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)


def _model(snap, dtype="f32"):
    from predicitivecoding_amd import PcDeviceModel
    return PcDeviceModel(snap, dtype)


def _one_hot(idx, n):
    y = np.zeros((len(idx), n), np.float32)
    y[np.arange(len(idx)), idx] = 1.0
    return y


def _check_classes(cls, rcls, rce, tol):
    srt = np.sort(rce.astype(np.float64), axis=1)
    margin = (srt[:, 1] - srt[:, 0]) if rce.shape[1] > 1 else np.full(len(rcls), np.inf)
    decided = margin > tol * (1 + np.abs(srt[:, 0]))
    assert np.array_equal(cls[decided], rcls[decided]), (cls, rcls)
    return int(decided.sum())


@pytest.mark.parametrize("act", ["tanh", "gelu", "sigmoid", "relu", "linear"])
@pytest.mark.parametrize("ffg", [False, True])
def test_clamped_relax_fp32(oracle, act, ffg):
    snap, W, b, P, x = build_case([37, 70, 19, 6], act, 0.1, batch=11, bias_scale=0.2, seed=7, ffg=ffg)
    top = make_inputs(11, 6, seed=8)
    m = _model(snap)
    try:
        st, en = m.relax_clamped(x, top, 10, want_states=True)
    finally:
        m.close()
    rst, ren = oracle.clamped_relax(snap.layer_sizes, act, 0.1, W, b, P, x, top, 10, ffg=ffg)
    errs = dict(energy=max_rel(en, ren), states=max(max_rel(a, r) for a, r in zip(st, rst)))
    _report(f"clamped/{act}/ffg={ffg}", **errs)
    assert np.array_equal(st[-1], top)
    assert all(v < 1e-4 for v in errs.values()), errs


def test_clamped_two_level_network_energy_only(oracle):
    # no free layer at all: the energy is the input's reconstruction error at every step
    snap, W, b, P, x = build_case([9, 4], "tanh", 0.1, batch=5, bias_scale=0.3, seed=9)
    top = make_inputs(5, 4, seed=10)
    m = _model(snap)
    try:
        _, en = m.relax_clamped(x, top, 3)
    finally:
        m.close()
    _, ren = oracle.clamped_relax([9, 4], "tanh", 0.1, W, b, P, x, top, 3)
    assert max_rel(en, ren) < 1e-4


@pytest.mark.parametrize("tile", [0, 32, 64, 128, 256])
def test_classify_c1_shape_fp32(oracle, tile):
    # the reference's MNIST-shaped classifier ([784,256,256,10] tanh) on a batch of 24
    snap, W, b, P, x = build_case([784, 256, 256, 10], "tanh", 0.1, batch=24, xdist="uniform01", seed=0)
    m = _model(snap)
    try:
        if tile:
            m.set_option("tile", tile)
        ce, cls, be = m.classify(x, 12)
    finally:
        m.close()
    rce, rcls, rbe = oracle.classify(snap.layer_sizes, "tanh", 0.1, W, b, P, x, 12)
    errs = dict(class_energies=max_rel(ce, rce), best_energy=max_rel(be, rbe))
    n = _check_classes(cls, rcls, rce, 1e-4)
    _report(f"classify c1 tile={tile} decided={n}/24", **errs)
    assert all(v < 1e-4 for v in errs.values()), errs
    assert np.array_equal(be, ce[np.arange(24), cls])


@pytest.mark.parametrize("act,ffg,act_reg", [("gelu", False, 0.0), ("sigmoid", True, 0.0), ("tanh", False, 0.01)])
def test_classify_options_fp32(oracle, act, ffg, act_reg):
    snap, W, b, P, x = build_case([29, 45, 33, 7], act, 0.15, batch=9, bias_scale=0.2, seed=12, ffg=ffg,
                                  act_reg=act_reg, precisions=[1.0, 0.8, 1.2, 1.0])
    m = _model(snap)
    try:
        ce, cls, be = m.classify(x, 9)
    finally:
        m.close()
    rce, rcls, rbe = oracle.classify(snap.layer_sizes, act, 0.15, W, b, P, x, 9, act_reg=act_reg, ffg=ffg)
    errs = dict(class_energies=max_rel(ce, rce), best_energy=max_rel(be, rbe))
    _check_classes(cls, rcls, rce, 1e-4)
    _report(f"classify {act} ffg={ffg} lam={act_reg}", **errs)
    assert all(v < 1e-4 for v in errs.values()), errs


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_classify_16bit_operands(oracle, dtype):
    snap, W, b, P, x = build_case([96, 130, 64, 12], "gelu", 0.05, batch=10, init="fanin", seed=13)
    m = _model(snap, dtype)
    try:
        ce, cls, be = m.classify(x, 8)
    finally:
        m.close()
    rce, rcls, _ = oracle.classify(snap.layer_sizes, "gelu", 0.05, W, b, P, x, 8, round_mode=ROUND[dtype])
    err = max_rel(ce, rce)
    _check_classes(cls, rcls, rce, 2e-3)
    _report(f"classify {dtype}", class_energies=err)
    assert err < 2e-3


def test_classify_graph_and_eager_agree_bit_for_bit():
    snap, _, _, _, x = build_case([40, 33, 8], "tanh", 0.1, batch=6, seed=14)
    m = _model(snap)
    try:
        g = m.classify(x, 7)
        m.set_option("use_graph", 0)
        e = m.classify(x, 7)
    finally:
        m.close()
    for a, b in zip(g, e):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("batch,wd", [(1, 0.0), (5, 0.0), (70, 0.01), (512, 0.0), (600, 0.01)])
def test_learn_step_fp32(oracle, batch, wd):
    # up to 512 rows the weights are updated by the one-launch small-batch
    # kernel (70 and 512 rows: several 64-row chunks), beyond by the grouped GEMM
    sizes = [37, 70, 19, 6]
    snap, W, b, P, x = build_case(sizes, "tanh", 0.1, batch=batch, bias_scale=0.1, seed=15)
    y = _one_hot(np.arange(batch) % 6, 6)
    m = _model(snap)
    try:
        en = m.learn(x, y, 9, 0.05, wd)
        gw, gb = m.get_weights()
        # the settling after the step uses the updated weights and W^T
        _, en2 = m.relax_clamped(x, y, 6)
    finally:
        m.close()
    rw, rb, ren = oracle.learn(sizes, "tanh", 0.1, W, b, P, x, y, 9, 0.05, weight_decay=wd)
    _, ren2 = oracle.clamped_relax(sizes, "tanh", 0.1, rw, rb, P, x, y, 6)
    errs = dict(weights=max(max_rel(a, r) for a, r in zip(gw, rw)), biases=max(max_rel(a, r) for a, r in zip(gb, rb)),
                energy=max_rel(en, ren), energy_after=max_rel(en2, ren2))
    _report(f"learn B={batch} wd={wd}", **errs)
    assert all(v < 1e-4 for v in errs.values()), errs


def test_train_two_patterns_then_predict(oracle):
    # AdaptiveInferenceTests.TrainTwoPatterns on the device ([4,8,2] tanh, eta 0.1,
    # eta_w 0.01, 40 epochs of Learn(a, 0), Learn(b, 1) with T = 30), checked
    # against the same sequence on the oracle, then classified (PredictWithEnergy).
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    from predicitivecoding_amd import GenerativeSnapshot
    snap = GenerativeSnapshot(sizes, ACT["tanh"], 0.1, 0.0, False, W, b, list(P))
    a = np.array([[1, 0, 0, 0]], np.float32)
    bb = np.array([[0, 0, 0, 1]], np.float32)
    m = _model(snap)
    rw, rb = W, b
    try:
        for _ in range(40):
            m.learn(a, _one_hot([0], 2), 30, 0.01)
            m.learn(bb, _one_hot([1], 2), 30, 0.01)
            rw, rb, _ = oracle.learn(sizes, "tanh", 0.1, rw, rb, P, a, _one_hot([0], 2), 30, 0.01)
            rw, rb, _ = oracle.learn(sizes, "tanh", 0.1, rw, rb, P, bb, _one_hot([1], 2), 30, 0.01)
        gw, gb = m.get_weights()
        ce, cls, be = m.classify(np.concatenate([a, bb]), 15)
    finally:
        m.close()
    werr = max(max_rel(g, r) for g, r in zip(gw + gb, rw + rb))
    _report("two patterns", weights=werr)
    assert werr < 1e-4
    assert list(cls) == [0, 1]
    rce, rcls, _ = oracle.classify(sizes, "tanh", 0.1, rw, rb, P, np.concatenate([a, bb]), 15)
    assert max_rel(ce, rce) < 1e-4 and list(rcls) == [0, 1]


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("batch", [9, 600])
def test_learn_step_16bit_masters(oracle, dtype, batch):
    # LearnMixed's scheme: 16-bit settling, fp32 master update, operands
    # re-rounded; a batch of 9 takes the one-launch small-batch update, 600 the
    # grouped GEMM
    sizes = [37, 70, 19, 6]
    snap, W, b, P, x = build_case(sizes, "gelu", 0.1, batch=batch, bias_scale=0.1, seed=17)
    y = _one_hot(np.arange(batch) % 6, 6)
    m = _model(snap, dtype)
    try:
        en = m.learn(x, y, 8, 0.05)
        gw, gb = m.get_weights()
        _, en2 = m.relax_clamped(x, y, 5)
    finally:
        m.close()
    rw, rb, ren = oracle.learn(sizes, "gelu", 0.1, W, b, P, x, y, 8, 0.05, round_mode=dtype)
    _, ren2 = oracle.clamped_relax(sizes, "gelu", 0.1, rw, rb, P, x, y, 5, round_mode=dtype)
    errs = dict(weights=max(max_rel(a, r) for a, r in zip(gw, rw)), biases=max(max_rel(a, r) for a, r in zip(gb, rb)),
                energy=max_rel(en, ren), energy_after=max_rel(en2, ren2))
    _report(f"learn {dtype}", **errs)
    assert all(v < 2e-3 for v in errs.values()), errs


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-4), ("bf16", 2e-3)])
def test_learn_step_c2_network(oracle, dtype, tol):
    # one learning step on BASELINE configs[1]'s network (1024-1024-1024-1024-256 tanh, eta 0.05)
    # with a batch of 64 labelled rows and T = 20, against the oracle's Learn (same operand rounding)
    sizes = [1024, 1024, 1024, 1024, 256]
    snap, W, b, P, x = build_case(sizes, "tanh", 0.05, batch=64, seed=25)
    y = _one_hot(np.arange(64) % 256, 256)
    m = _model(snap, dtype)
    try:
        en = m.learn(x, y, 20, 0.01, 0.001)
        gw, gb = m.get_weights()
    finally:
        m.close()
    rw, rb, ren = oracle.learn(sizes, "tanh", 0.05, W, b, P, x, y, 20, 0.01, weight_decay=0.001,
                               round_mode=ROUND[dtype])
    errs = dict(weights=max(max_rel(a, r) for a, r in zip(gw, rw)), biases=max(max_rel(a, r) for a, r in zip(gb, rb)),
                energy=max_rel(en, ren),
                update=max(max_rel(a - w0, r - w0) for a, r, w0 in zip(gw, rw, W)))
    _report(f"learn c2 network {dtype}", **errs)
    assert all(v < tol for v in errs.values()), errs


def test_learn_mixed_predicts_like_float(oracle):
    # NetworkTests' mixed-precision contract: the bf16 model trained with
    # LearnMixed's scheme classifies the two patterns like the fp32 network
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    from predicitivecoding_amd import GenerativeSnapshot
    snap = GenerativeSnapshot(sizes, ACT["tanh"], 0.1, 0.0, False, W, b, list(P))
    a = np.array([[1, 0, 0, 0]], np.float32)
    bb = np.array([[0, 0, 0, 1]], np.float32)
    m = _model(snap, "bf16")
    try:
        for _ in range(40):
            m.learn(a, _one_hot([0], 2), 30, 0.01)
            m.learn(bb, _one_hot([1], 2), 30, 0.01)
        gw, _ = m.get_weights()
        _, cls, _ = m.classify(np.concatenate([a, bb]), 15)
    finally:
        m.close()
    assert list(cls) == [0, 1]
    assert all(np.all(np.isfinite(w)) for w in gw)


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-4), ("bf16", 2e-3)])
def test_learn_from_hidden_states(oracle, dtype, tol):
    # pcd_pc_learn_warm: the settling starts from given hidden states (the Mu a
    # reference network holds between Learn calls) and returns the settled ones
    sizes = [37, 70, 19, 6]
    snap, W, b, P, x = build_case(sizes, "tanh", 0.1, batch=7, bias_scale=0.1, seed=19)
    y = _one_hot(np.arange(7) % 6, 6)
    rng = np.random.default_rng(20)
    hidden = [(rng.standard_normal((7, s)) * 0.4).astype(np.float32) for s in sizes[1:-1]]
    m = _model(snap, dtype)
    try:
        # one array too many (or too few) is refused before anything runs,
        # not truncated to the hidden layer count
        for wrong in (hidden + [hidden[0]], hidden[:1]):
            with pytest.raises(ArgumentException):
                m.learn(x, y, 9, 0.05, hidden=wrong)
        en, gh = m.learn(x, y, 9, 0.05, hidden=hidden, want_hidden=True)
        gw, gb = m.get_weights()
    finally:
        m.close()
    rw, rb, ren, rh = oracle.learn(sizes, "tanh", 0.1, W, b, P, x, y, 9, 0.05, round_mode=ROUND[dtype],
                                   hidden=hidden, want_hidden=True)
    errs = dict(weights=max(max_rel(a, r) for a, r in zip(gw, rw)), biases=max(max_rel(a, r) for a, r in zip(gb, rb)),
                energy=max_rel(en, ren), hidden=max(max_rel(a, r) for a, r in zip(gh, rh)))
    _report(f"learn warm {dtype}", **errs)
    assert all(v < tol for v in errs.values()), errs


def test_train_two_patterns_with_carried_hidden_state(oracle):
    # TrainTwoPatterns as the reference runs it on one network: each Learn
    # starts from the hidden state the previous one settled to (Network.cs:143,
    # 150-151).  Device chain against the oracle chain, call after call.
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    from predicitivecoding_amd import GenerativeSnapshot
    snap = GenerativeSnapshot(sizes, ACT["tanh"], 0.1, 0.0, False, W, b, list(P))
    a = np.array([[1, 0, 0, 0]], np.float32)
    bb = np.array([[0, 0, 0, 1]], np.float32)
    m = _model(snap)
    rw, rb, rh = W, b, None
    gh = None
    worst = 0.0
    try:
        for _ in range(40):
            for x, y in ((a, _one_hot([0], 2)), (bb, _one_hot([1], 2))):
                _, gh = m.learn(x, y, 30, 0.01, hidden=gh, want_hidden=True)
                rw, rb, _, rh = oracle.learn(sizes, "tanh", 0.1, rw, rb, P, x, y, 30, 0.01, hidden=rh,
                                             want_hidden=True)
                worst = max(worst, max_rel(gh[0], rh[0]))
        gw, gb = m.get_weights()
        _, cls, _ = m.classify(np.concatenate([a, bb]), 15)
    finally:
        m.close()
    werr = max(max_rel(g, r) for g, r in zip(gw + gb, rw + rb))
    _report("two patterns, carried hidden state", weights=werr, hidden=worst)
    assert werr < 1e-4 and worst < 1e-4
    assert list(cls) == [0, 1]
