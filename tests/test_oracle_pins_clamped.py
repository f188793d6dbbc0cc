"""Pins of the oracle's clamped-top settling, minimum-energy classification and
learning step (oracle/pc_oracle.c: pco_clamped_relax, pco_classify, pco_learn).

Each is checked against something that shares no code with it: torch autograd
of the free energy with the top held fixed (and autograd of the
pre-activation for the learning signal), the closed-form solution of the
linear network with both ends clamped, and the behaviours the reference's own
tests assert after training (AdaptiveInferenceTests.cs, NetworkTests.cs).
"""
import numpy as np
import pytest

from tests.autograd_ref import autograd_learn, autograd_relax
from tests.netgen import close, make_inputs, make_net

ACTS = ["linear", "tanh", "relu", "sigmoid", "gelu"]


def one_hot(idx, n):
    y = np.zeros((len(idx), n), np.float32)
    y[np.arange(len(idx)), idx] = 1.0
    return y


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("ffg", [False, True])
def test_clamped_relax_matches_autograd(oracle, act, ffg):
    sizes = [7, 9, 5, 4]
    W, b, _ = make_net(sizes, seed=21, bias_scale=0.2)
    P = [1.0, 0.8, 1.3, 1.0]
    x = make_inputs(4, 7, seed=22)
    top = make_inputs(4, 4, seed=23)
    T = 8
    _, st_ref, en_ref = autograd_relax(sizes, act, 0.1, W, b, P, x, T, ffg=ffg, top_clamp=top)
    _, st64, en64 = oracle.persample_relax_f64(sizes, act, 0.1, W, b, P, x, T, ffg=ffg, top_clamp=top,
                                               want_states=True, want_energy=True)
    for l in range(len(sizes)):
        assert np.max(np.abs(st64[l] - st_ref[l])) < 1e-10
    assert np.max(np.abs(en64 - en_ref)) < 1e-10
    assert np.array_equal(st64[-1], top.astype(np.float64))     # the clamp holds
    st32, en32 = oracle.clamped_relax(sizes, act, 0.1, W, b, P, x, top, T, ffg=ffg)
    for l in range(len(sizes)):
        assert close(st32[l], st_ref[l], 1e-5)
    assert close(en32, en_ref, 1e-5)


def test_clamped_linear_closed_form(oracle):
    # Linear f, input and top clamped, one free layer mu1:
    #   mu1' = A mu1 + c,  A = I - eta (P1 I + P0 W1'W1),  c = eta (P0 W1'(x - b1) + P1 (W2 y + b2))
    # so from mu1 = 0, mu1_T = (I - A)^-1 (I - A^T) c.
    sizes = [10, 6, 3]
    W, b, _ = make_net(sizes, seed=31, bias_scale=0.3)
    x = make_inputs(3, 10, seed=32).astype(np.float64)
    y = make_inputs(3, 3, seed=33).astype(np.float64)
    P0, P1, eta, T = 1.2, 0.7, 0.08, 40
    W1, W2 = W[0].astype(np.float64), W[1].astype(np.float64)
    b1, b2 = b[0].astype(np.float64), b[1].astype(np.float64)
    A = np.eye(6) - eta * (P1 * np.eye(6) + P0 * W1.T @ W1)
    G = np.linalg.solve(np.eye(6) - A, np.eye(6) - np.linalg.matrix_power(A, T))
    _, st, en = oracle.persample_relax_f64(sizes, "linear", eta, W, b, [P0, P1, 1.0], x, T, top_clamp=y,
                                           want_states=True, want_energy=True)
    for i in range(3):
        c = eta * (P0 * W1.T @ (x[i] - b1) + P1 * (W2 @ y[i] + b2))
        mu = G @ c
        assert np.max(np.abs(st[1][i] - mu)) < 1e-10
        # energy of the last step is read at mu_{T-1}
        Gm = np.linalg.solve(np.eye(6) - A, np.eye(6) - np.linalg.matrix_power(A, T - 1))
        m1 = Gm @ c
        r0 = x[i] - W1 @ m1 - b1
        r1 = m1 - W2 @ y[i] - b2
        want = 0.5 * P0 * r0 @ r0 + 0.5 * P1 * r1 @ r1
        assert abs(en[T - 1, i] - want) < 1e-10
    st32, en32 = oracle.clamped_relax(sizes, "linear", eta, W, b, [P0, P1, 1.0], x, y, T)
    assert close(st32[1], st[1], 1e-5) and close(en32, en, 1e-5)


@pytest.mark.parametrize("act", ["tanh", "gelu", "sigmoid"])
def test_classify_matches_autograd_per_class(oracle, act):
    # PredictCore: C settlings per sample with the top clamped to one-hot(c),
    # F(x, c) the last step's energy, first minimum wins.
    sizes = [6, 8, 5]
    W, b, P = make_net(sizes, seed=41, bias_scale=0.1)
    x = make_inputs(4, 6, seed=42)
    T, C = 12, 5
    ce, bc, be = oracle.classify(sizes, act, 0.1, W, b, P, x, T)
    want = np.zeros((4, C))
    for c in range(C):
        _, _, en = autograd_relax(sizes, act, 0.1, W, b, P, x, T, top_clamp=one_hot([c] * 4, C))
        want[:, c] = en[-1]
    assert close(ce, want, 1e-5)
    assert np.array_equal(bc, np.argmin(ce, axis=1))            # numpy argmin takes the first minimum too
    assert np.array_equal(be, ce[np.arange(4), bc])


def test_classify_first_minimum_wins_ties(oracle):
    # Zero weights and biases: F(x, c) = 0.5 |x|^2 for every c, so class 0 wins (strict <).
    sizes = [4, 3, 3]
    W = [np.zeros((4, 3), np.float32), np.zeros((3, 3), np.float32)]
    b = [np.zeros(4, np.float32), np.zeros(3, np.float32)]
    x = np.array([[1.0, -2.0, 0.5, 0.0]], np.float32)
    ce, bc, be = oracle.classify(sizes, "tanh", 0.1, W, b, [1.0] * 3, x, 5)
    assert np.all(ce == ce[0, 0]) and bc[0] == 0
    assert abs(be[0] - 0.5 * np.sum(x.astype(np.float64) ** 2)) < 1e-6


@pytest.mark.parametrize("act,wd", [("tanh", 0.0), ("gelu", 0.0), ("sigmoid", 0.01), ("linear", 0.02)])
def test_learn_matches_autograd(oracle, act, wd):
    sizes = [6, 9, 4]
    W, b, P = make_net(sizes, seed=51, bias_scale=0.1)
    x = make_inputs(5, 6, seed=52)
    y = one_hot([0, 3, 1, 2, 3], 4)
    T, eta_w = 10, 0.05
    nw, nb, en = oracle.learn(sizes, act, 0.1, W, b, P, x, y, T, eta_w, weight_decay=wd)
    rw, rb, ren = autograd_learn(sizes, act, 0.1, W, b, P, x, y, T, eta_w, weight_decay=wd)
    for l in range(len(nw)):
        assert close(nw[l], rw[l], 1e-5)
        assert close(nb[l], rb[l], 1e-5)
        # and the update is not vacuous
        assert np.max(np.abs(rw[l] - W[l])) > 1e-4
    assert close(en, ren, 1e-5)


def test_learn_batch_is_sum_of_single_sample_updates(oracle):
    sizes = [5, 7, 3]
    W, b, P = make_net(sizes, seed=61, bias_scale=0.1)
    x = make_inputs(3, 5, seed=62)
    y = one_hot([2, 0, 1], 3)
    nw, nb, _ = oracle.learn(sizes, "tanh", 0.1, W, b, P, x, y, 8, 0.1)
    acc_w = [w.astype(np.float64).copy() for w in W]
    acc_b = [v.astype(np.float64).copy() for v in b]
    for i in range(3):
        w1, b1, _ = oracle.learn(sizes, "tanh", 0.1, W, b, P, x[i:i + 1], y[i:i + 1], 8, 0.1)
        for l in range(2):
            acc_w[l] += w1[l] - W[l]
            acc_b[l] += b1[l] - b[l]
    for l in range(2):
        assert close(nw[l], acc_w[l], 1e-5) and close(nb[l], acc_b[l], 1e-5)


def _train_two_patterns(oracle, sizes, eta, eta_w, epochs, T, W, b, P):
    # AdaptiveInferenceTests.TrainTwoPatterns: Learn(a, 0), Learn(b, 1), sequentially
    a = np.array([[1, 0, 0, 0]], np.float32)
    bb = np.array([[0, 0, 0, 1]], np.float32)
    for _ in range(epochs):
        W, b, _ = oracle.learn(sizes, "tanh", eta, W, b, P, a, one_hot([0], 2), T, eta_w)
        W, b, _ = oracle.learn(sizes, "tanh", eta, W, b, P, bb, one_hot([1], 2), T, eta_w)
    return W, b, a, bb


def test_trained_two_patterns_classify_correctly(oracle):
    # AdaptiveInferenceTests.cs:117-129 / NetworkTests.cs: after TrainTwoPatterns
    # ([4,8,2] tanh, eta 0.1, eta_w 0.01, 40 epochs of T = 30) each pattern is
    # classified as its own label.  Initial weights are this repository's seeded
    # Xavier draw, not .NET's Random(42).
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    W, b, a, bb = _train_two_patterns(oracle, sizes, 0.1, 0.01, 40, 30, W, b, P)
    ce, bc, be = oracle.classify(sizes, "tanh", 0.1, W, b, P, np.concatenate([a, bb]), 15)
    assert list(bc) == [0, 1]
    assert np.all(np.isfinite(be)) and np.all(be >= 0)


def test_trained_class_energies_mixed_track_float(oracle):
    # NetworkTests.cs:403-440 (ClassEnergiesMixed_TracksFloatEnergies_AndAgreesOnTheWinner):
    # [4,16,2] tanh, eta 0.2, eta_w 0.05, 200 epochs of T = 10 on x0 = 0 -> 0, x1 = 1 -> 1;
    # the half-precision class energies stay within 5e-2 (1 + |F|) and pick the same class.
    sizes = [4, 16, 2]
    W, b, P = make_net(sizes, seed=0)
    x0 = np.zeros((1, 4), np.float32)
    x1 = np.ones((1, 4), np.float32)
    for _ in range(200):
        W, b, _ = oracle.learn(sizes, "tanh", 0.2, W, b, P, x0, one_hot([0], 2), 10, 0.05)
        W, b, _ = oracle.learn(sizes, "tanh", 0.2, W, b, P, x1, one_hot([1], 2), 10, 0.05)
    xs = np.concatenate([x0, x1])
    full, bc, _ = oracle.classify(sizes, "tanh", 0.2, W, b, P, xs, 20)
    half, bch, _ = oracle.classify(sizes, "tanh", 0.2, W, b, P, xs, 20, round_mode="f16")
    assert np.all(np.abs(full - half) <= 5e-2 * (1 + np.abs(full)))
    assert list(bc) == list(bch) == [0, 1]


@pytest.mark.parametrize("mode", ["bf16", "f16"])
def test_mixed_learn_tracks_float_learn(oracle, mode):
    # LearnMixed differs from Learn only by the 16-bit settling (and its rounded
    # delta): the updated masters stay within half precision's tolerance
    sizes = [6, 9, 4]
    W, b, P = make_net(sizes, seed=71, bias_scale=0.1)
    x = make_inputs(5, 6, seed=72)
    y = one_hot([0, 3, 1, 2, 3], 4)
    fw, fb, fe = oracle.learn(sizes, "tanh", 0.1, W, b, P, x, y, 10, 0.05)
    mw, mb, me = oracle.learn(sizes, "tanh", 0.1, W, b, P, x, y, 10, 0.05, round_mode=mode)
    for l in range(2):
        assert close(mw[l], fw[l], 2e-2) and close(mb[l], fb[l], 2e-2)
        assert not np.array_equal(mw[l], fw[l])      # the rounding is really applied
    assert close(me, fe, 5e-2)


# ---------------------------------------------------- adaptive classification

def _exit_step_by_hand(trace, max_steps, eps):
    """SettleAdaptive's rule read off a fixed-step energy trace
    (Network.cs:895-905): the first step k >= 2 whose energy fell by less than
    eps * max(previous, 1e-12), in float arithmetic; max_steps if none."""
    if eps <= 0:
        return max_steps
    for k in range(1, max_steps):
        prev, cur = np.float32(trace[k - 1]), np.float32(trace[k])
        if prev - cur < np.float32(eps) * max(prev, np.float32(1e-12)):
            return k + 1
    return max_steps


@pytest.mark.parametrize("act,ffg", [("tanh", False), ("gelu", True), ("sigmoid", False)])
def test_classify_adaptive_exit_steps_by_hand(oracle, act, ffg):
    # Each candidate's steps and energy, recomputed from its own fixed-step
    # clamped settling (one-hot label, pco_clamped_relax) and the exit rule
    # applied by hand; the winner is the first minimum and its settling counts
    # twice (Network.cs:803-840).
    sizes = [12, 20, 9, 4]
    W, b, P = make_net(sizes, seed=51, bias_scale=0.2)
    x = make_inputs(5, 12, seed=52, dist="uniform01")
    T, C = 40, 4
    for eps in (3e-2, 1e-2, 1e-3):
        ce, cs, bc, be, su = oracle.classify_adaptive(sizes, act, 0.1, W, b, P, x, T, eps, ffg=ffg)
        fired = 0
        for i in range(len(x)):
            for c in range(C):
                _, tr = oracle.clamped_relax(sizes, act, 0.1, W, b, P, x[i:i + 1], one_hot([c], C), T, ffg=ffg)
                k = _exit_step_by_hand(tr[:, 0], T, eps)
                assert cs[i, c] == k, (eps, i, c, cs[i, c], k)
                assert ce[i, c] == pytest.approx(float(tr[k - 1, 0]), rel=1e-6)
                fired += k < T
            assert bc[i] == int(np.argmin(ce[i]))
            assert be[i] == ce[i, bc[i]]
            assert su[i] == cs[i].sum() + cs[i, bc[i]]
        assert fired > 0, eps


def test_classify_adaptive_epsilon_zero_is_predict_with_energy(oracle):
    # AdaptiveInferenceTests.cs:74-95: epsilon = 0 is PredictWithEnergy exactly,
    # with every candidate and the winner's re-run at the full budget
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    W, b, a, bb = _train_two_patterns(oracle, sizes, 0.1, 0.01, 40, 30, W, b, P)
    x = np.concatenate([a, bb])
    ce, bc, be = oracle.classify(sizes, "tanh", 0.1, W, b, P, x, 15)
    ace, acs, abc, abe, asu = oracle.classify_adaptive(sizes, "tanh", 0.1, W, b, P, x, 15, 0.0)
    assert np.array_equal(ce, ace) and np.array_equal(bc, abc) and np.array_equal(be, abe)
    assert np.all(acs == 15) and np.all(asu == 15 * (2 + 1))


def test_classify_adaptive_saves_steps_and_stays_correct(oracle):
    # AdaptiveInferenceTests.cs:116-131: a generous budget (200) and epsilon
    # 1e-3 after TrainTwoPatterns: pattern a is class 0, finite non-negative
    # energy, fewer than 200 * (2 + 1) steps spent.
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    W, b, a, bb = _train_two_patterns(oracle, sizes, 0.1, 0.01, 40, 30, W, b, P)
    _, cs, bc, be, su = oracle.classify_adaptive(sizes, "tanh", 0.1, W, b, P, np.concatenate([a, bb]), 200, 1e-3)
    assert list(bc) == [0, 1]
    assert np.all(np.isfinite(be)) and np.all(be >= 0)
    assert np.all(su < 200 * 3), su


def test_classify_adaptive_monotone_in_epsilon_and_budget_invariant(oracle):
    # AdaptiveInferenceTests.cs:97-114 applied per candidate: a looser epsilon
    # stops no later, and an exit inside the budget does not move when the
    # budget grows
    sizes = [10, 16, 6, 3]
    W, b, P = make_net(sizes, seed=61, bias_scale=0.1)
    x = make_inputs(6, 10, seed=62, dist="uniform01")
    _, loose, _, _, _ = oracle.classify_adaptive(sizes, "tanh", 0.1, W, b, P, x, 60, 1e-2)
    _, tight, _, _, _ = oracle.classify_adaptive(sizes, "tanh", 0.1, W, b, P, x, 60, 1e-4)
    _, wide, _, _, _ = oracle.classify_adaptive(sizes, "tanh", 0.1, W, b, P, x, 200, 1e-2)
    assert np.all(loose <= tight) and np.any(loose < 60)
    assert np.array_equal(loose[loose < 60], wide[loose < 60])


def test_effort_presets(oracle):
    # EffortPresets.For (EffortLevel.cs:33-39) and AdaptiveInferenceTests.cs:133-142:
    # steps grow and the tolerance tightens with the effort level
    low, med, high = (oracle.EFFORT_PRESETS[k] for k in ("low", "medium", "high"))
    assert (low, med, high) == ((10, 1e-3), (30, 1e-4), (100, 1e-5))
    assert low[0] < med[0] < high[0] and low[1] > med[1] > high[1]


# ------------------------------------------ learning from carried hidden states

@pytest.mark.parametrize("act", ["tanh", "gelu"])
def test_learn_from_hidden_states_matches_autograd(oracle, act):
    # Network.Learn settles from the hidden states the network holds
    # (ReadAllLayers, Network.cs:143; InferCore resets nothing), and persists
    # the settled ones (:150-151).  The oracle's warm-started step against the
    # float64 autograd statement started from the same states: weights, biases,
    # energies and the settled hidden states.
    sizes = [10, 14, 9, 3]
    W, b, P = make_net(sizes, seed=31, bias_scale=0.2)
    x = make_inputs(4, 10, seed=32, dist="uniform01")
    y = one_hot([0, 2, 1, 2], 3)
    rng = np.random.default_rng(33)
    hidden = [(rng.standard_normal((4, s)) * 0.5).astype(np.float32) for s in sizes[1:-1]]
    nw, nb, en, nh = oracle.learn(sizes, act, 0.1, W, b, P, x, y, 12, 0.05, hidden=hidden, want_hidden=True)
    rw, rb, ren, rh = autograd_learn(sizes, act, 0.1, W, b, P, x, y, 12, 0.05, init_hidden=hidden, want_hidden=True)
    for l in range(len(nw)):
        assert close(nw[l], rw[l], 1e-5) and close(nb[l], rb[l], 1e-5)
    assert close(en, ren, 1e-5)
    for a, c in zip(nh, rh):
        assert close(a, c, 1e-5)
    # the start matters: from zero the step is another one
    zw, _, _ = oracle.learn(sizes, act, 0.1, W, b, P, x, y, 12, 0.05)
    assert not close(zw[0], nw[0], 1e-3)
    # no hidden states given is a network at zero, bit for bit
    z2, _, _ = oracle.learn(sizes, act, 0.1, W, b, P, x, y, 12, 0.05,
                            hidden=[np.zeros((4, s), np.float32) for s in sizes[1:-1]])
    assert all(np.array_equal(a, c) for a, c in zip(zw, z2))


def test_train_two_patterns_with_carried_hidden_state(oracle):
    # AdaptiveInferenceTests.TrainTwoPatterns as the reference runs it: Learn(a,
    # 0), Learn(b, 1), ... on one network, each call starting from the hidden
    # state the previous one settled to.  The oracle's chain with the state
    # carried equals the autograd chain with the state carried, call after
    # call; and it is not the chain that restarts every call from zero.
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42)
    a = np.array([[1, 0, 0, 0]], np.float32)
    bb = np.array([[0, 0, 0, 1]], np.float32)
    ow, ob, oh = W, b, [np.zeros((1, 8), np.float32)]
    rw, rb, rh = [w.astype(np.float64) for w in W], [v.astype(np.float64) for v in b], [np.zeros((1, 8))]
    zw, zb = W, b
    for _ in range(6):
        for x, y in ((a, one_hot([0], 2)), (bb, one_hot([1], 2))):
            ow, ob, _, oh = oracle.learn(sizes, "tanh", 0.1, ow, ob, P, x, y, 30, 0.01, hidden=oh, want_hidden=True)
            rw, rb, _, rh = autograd_learn(sizes, "tanh", 0.1, rw, rb, P, x, y, 30, 0.01, init_hidden=rh,
                                           want_hidden=True)
            zw, zb, _ = oracle.learn(sizes, "tanh", 0.1, zw, zb, P, x, y, 30, 0.01)
            for l in range(2):
                assert close(ow[l], rw[l], 1e-5) and close(ob[l], rb[l], 1e-5)
            assert close(oh[0], rh[0], 1e-5)
    assert not close(ow[0], zw[0], 1e-4)
