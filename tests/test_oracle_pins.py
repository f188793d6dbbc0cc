"""Pins of the CPU oracle (oracle/pc_oracle.c) before anything is checked against it.

Each test checks the oracle against something that does not share its code:
the closed forms the reference's own tests assert, independent library
routines (torch / numpy rounding and GELU), torch autograd of the free energy,
and closed-form solutions of the linear relaxation.
"""
import math

import numpy as np
import pytest
import torch

from tests.autograd_ref import autograd_relax
from tests.netgen import close, make_inputs, make_net, max_rel

ACTS = ["linear", "tanh", "relu", "sigmoid", "gelu"]


# ---------------------------------------------------------------- activations

def test_activation_closed_forms(oracle):
    # ActivationFnTests.cs:21-28 (tanh), :31-38 (relu), :41-49 (sigmoid)
    z = oracle.act_apply("tanh", [0.0, 1.0, -1.0])
    assert z[0] == 0.0 and abs(z[1] - math.tanh(1)) < 1e-6 and abs(z[2] - math.tanh(-1)) < 1e-6
    z = oracle.act_apply("relu", [-2.0, 0.0, 3.0])
    assert list(z) == [0.0, 0.0, 3.0]
    z = oracle.act_apply("sigmoid", [-3.0, 0.0, 3.0])
    assert 0 < z[0] < 0.5 and abs(z[1] - 0.5) < 1e-7 and 0.5 < z[2] < 1
    assert list(oracle.act_apply("linear", [-1.0, 0.0, 1.0, 2.0])) == [-1.0, 0.0, 1.0, 2.0]


def test_activation_derivative_closed_forms(oracle):
    # ActivationFnTests.cs:54-90
    assert np.all(oracle.act_deriv("linear", [-1.0, 0.0, 2.0]) == 1.0)
    d = oracle.act_deriv("tanh", [0.0, 1.0])
    assert abs(d[0] - 1.0) < 1e-7 and abs(d[1] - (1 - math.tanh(1) ** 2)) < 1e-6
    assert list(oracle.act_deriv("relu", [-1.0, 0.0, 1.0])) == [0.0, 0.0, 1.0]
    d = oracle.act_deriv("sigmoid", [0.0, 2.0])
    s2 = 1 / (1 + math.exp(-2))
    assert abs(d[0] - 0.25) < 1e-7 and abs(d[1] - s2 * (1 - s2)) < 1e-6


def test_gelu_matches_torch_tanh_gelu(oracle):
    x = np.linspace(-8, 8, 4001)
    ref = torch.nn.functional.gelu(torch.tensor(x), approximate="tanh").numpy()
    assert np.max(np.abs(oracle.act_apply("gelu", x, np.float64) - ref)) < 1e-12
    assert np.max(np.abs(oracle.act_apply("gelu", x, np.float32) - ref)) < 2e-6


@pytest.mark.parametrize("act", ACTS)
def test_derivative_matches_autograd(oracle, act):
    x = np.linspace(-5, 5, 2001)
    x = x[np.abs(x) > 1e-3]  # ReLU kink
    xt = torch.tensor(x, requires_grad=True)
    from tests.autograd_ref import _act
    (g,) = torch.autograd.grad(_act(act)(xt).sum(), xt)
    assert np.max(np.abs(oracle.act_deriv(act, x, np.float64) - g.numpy())) < 1e-12
    assert np.max(np.abs(oracle.act_deriv(act, x, np.float32) - g.numpy())) < 5e-6


# ------------------------------------------------------------------- rounding

def test_bf16_reference_values(oracle):
    # MixedSub16Tests.cs:35-56: round-trip within |x|/128, NaN kept, idempotent
    v = np.array([0, 1, -1, 0.1, -3.7, 1e-3, 12345.678, -6.5e4, 3e30, np.nan], dtype=np.float32)
    back = oracle.round16("bf16", v)
    fin = np.isfinite(v)
    assert np.all(np.abs(back[fin] - v[fin]) <= np.abs(v[fin]) / 128)
    assert np.isnan(back[-1])
    assert np.array_equal(oracle.bf16_bits(back), oracle.bf16_bits(v))


def test_bf16_matches_torch_rne(oracle):
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 200000),
        # exact ties: low 16 bits 0x8000 with even and odd kept bit
        (np.arange(1, 5001, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ]).astype(np.float32)
    ours = oracle.round16("bf16", v)
    ref = torch.tensor(v).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(1)
    v = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 18, 200000),
        np.array([65504, 65519.99, 65520, 70000, -1e9, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0, -0.0], np.float32),
        (np.arange(1, 5001, dtype=np.uint32) << 13 | 0x1000 | (120 << 23)).view(np.float32),  # ties
    ]).astype(np.float32)
    ours = oracle.round16("f16", v)
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).astype(np.float32)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


# ----------------------------------------------------------------------- GEMM

def test_gemm_known_answer(oracle):
    # LlmDeviceTests.cs:41-55: [1 2 3;4 5 6]·[7 8;9 10;11 12] = [58 64;139 154]
    c = oracle.gemm(np.array([[1, 2, 3], [4, 5, 6]]), np.array([[7, 8], [9, 10], [11, 12]]))
    assert c.tolist() == [[58, 64], [139, 154]]
    # TensorUtilsTests.cs:25-51: W v = [3, 7], W^T v = [4, 6]
    W = np.array([[1, 2], [3, 4]], dtype=np.float32)
    assert oracle.gemm(np.ones((1, 2)), W.T).ravel().tolist() == [3, 7]
    assert oracle.gemm(np.ones((1, 2)), W).ravel().tolist() == [4, 6]


def test_gemm_random_and_mixed(oracle):
    rng = np.random.default_rng(2)
    a = rng.standard_normal((37, 53)).astype(np.float32)
    b = rng.standard_normal((53, 29)).astype(np.float32)
    a[3, 5] = 0.0
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(oracle.gemm(a, b) - exact)) < 1e-4
    # MixedGemmTests.cs:20-41: 16-bit operands within 1e-2*(1+|x|) of float on 8x16x4
    a8, b8 = rng.random((8, 16)).astype(np.float32), rng.random((16, 4)).astype(np.float32)
    for mode in ("f16", "bf16"):
        assert close(oracle.gemm(a8, b8, mode), oracle.gemm(a8, b8), 1e-2)
        # the rounding happens on the operands only
        ar, br = oracle.round16(mode, a), oracle.round16(mode, b)
        assert np.max(np.abs(oracle.gemm(a, b, mode) - ar.astype(np.float64) @ br.astype(np.float64))) < 1e-4


# ---------------------------------------------------------- relaxation pins

def test_energy_closed_form_first_step(oracle):
    # Layer.LocalEnergy 0.5*(9+16)=12.5 (PCLayerTests.cs:98-107): linear 2-layer
    # net, mu_1 = 0 so pred = b, e_0 = x - b = [3, 4].
    sizes = [2, 3]
    W = [np.array([[0.5, -1.0, 2.0], [1.5, 0.25, -0.5]], np.float32)]
    b = [np.array([1.0, 2.0], np.float32)]
    x = np.array([[4.0, 6.0]], np.float32)
    for fn in (oracle.batched_relax,):
        top, _, en = fn(sizes, "linear", 0.1, W, b, [1, 1], x, 1, want_energy=True)
        assert abs(en[0, 0] - 12.5) < 1e-6
        # T=1 from zero: mu_top = eta * W^T (f'(b) . P0 (x - f(b)))
        assert np.allclose(top[0], 0.1 * W[0].T @ np.array([3.0, 4.0]), atol=1e-6)


@pytest.mark.parametrize("act", ACTS)
def test_first_step_closed_form(oracle, act):
    # T=1 from zero state, 2 layers: top = eta * W^T [f'(b) . P0 (x - f(b))]
    sizes = [7, 5]
    W, b, _ = make_net(sizes, seed=3, bias_scale=0.5)
    x = make_inputs(4, 7, seed=4)
    P0 = 1.7
    pre = b[0].astype(np.float64)
    from tests.autograd_ref import _act
    bt = torch.tensor(pre, requires_grad=True)
    y = _act(act)(bt)
    (fp,) = torch.autograd.grad(y.sum(), bt)
    want = 0.05 * (P0 * (x - y.detach().numpy()) * fp.numpy()) @ W[0].astype(np.float64)
    top, _, _ = oracle.persample_relax_f64(sizes, act, 0.05, W, b, [P0, 1.0], x, 1)
    assert np.max(np.abs(top - want)) < 1e-12
    top32, _, _ = oracle.batched_relax(sizes, act, 0.05, W, b, [P0, 1.0], x, 1)
    assert np.max(np.abs(top32 - want)) < 1e-5


def test_linear_two_layer_closed_form(oracle):
    # Linear f, one free layer: Richardson iteration on least squares,
    # mu_T = (I - (I - eta P0 A)^T) A^-1 W^T (x - b),  A = W^T W.
    sizes = [12, 5]
    W, b, _ = make_net(sizes, seed=5, bias_scale=0.3)
    x = make_inputs(3, 12, seed=6).astype(np.float64)
    eta, P0, T = 0.07, 1.3, 25
    Wd = W[0].astype(np.float64)
    A = Wd.T @ Wd
    M = np.eye(5) - np.linalg.matrix_power(np.eye(5) - eta * P0 * A, T)
    want = (M @ np.linalg.solve(A, Wd.T @ (x - b[0]).T)).T
    top, _, en = oracle.persample_relax_f64(sizes, "linear", eta, W, b, [P0, 1.0], x, T, want_energy=True)
    assert np.max(np.abs(top - want)) < 1e-10
    # energy at step t is 0.5*P0*|x - b - W mu_t|^2 of the pre-update state
    mu = np.zeros((3, 5))
    for t in range(T):
        r = x - b[0] - mu @ Wd.T
        assert np.allclose(en[t], 0.5 * P0 * (r * r).sum(1), rtol=1e-12, atol=1e-12)
        mu = mu + eta * P0 * r @ Wd
    top32, _, _ = oracle.batched_relax(sizes, "linear", eta, W, b, [P0, 1.0], x, T)
    assert close(top32, want, 1e-5)


def test_linear_deep_closed_form(oracle):
    # Deeper linear nets are gradient descent on a quadratic F(z) = 0.5 z'Hz - g'z
    # (block-tridiagonal H): from z_0 = 0, z_T = (I - (I - eta H)^T) H^-1 g.
    sizes = [9, 6, 4]
    W, b, _ = make_net(sizes, seed=7, init=0.3, bias_scale=0.2)
    x = make_inputs(2, 9, seed=8).astype(np.float64)
    P = [1.0, 0.8, 1.0]
    eta, T = 0.2, 150
    W1, W2 = W[0].astype(np.float64), W[1].astype(np.float64)
    b1, b2 = b[0].astype(np.float64), b[1].astype(np.float64)
    n1, n2 = 6, 4
    H = np.zeros((n1 + n2, n1 + n2))
    H[:n1, :n1] = P[0] * W1.T @ W1 + P[1] * np.eye(n1)
    H[:n1, n1:] = -P[1] * W2
    H[n1:, :n1] = -P[1] * W2.T
    H[n1:, n1:] = P[1] * W2.T @ W2
    G = np.eye(n1 + n2) - np.linalg.matrix_power(np.eye(n1 + n2) - eta * H, T)
    for i in range(2):
        g = np.concatenate([P[0] * W1.T @ (x[i] - b1) + P[1] * b2, -P[1] * W2.T @ b2])
        z = G @ np.linalg.solve(H, g)
        top, st, _ = oracle.persample_relax_f64(sizes, "linear", eta, W, b, P, x[i:i + 1], T, want_states=True)
        assert np.max(np.abs(st[1][0] - z[:n1])) < 1e-10
        assert np.max(np.abs(top[0] - z[n1:])) < 1e-10


def test_activity_regularisation_energy_trace(oracle):
    sizes = [3, 4, 2]
    W = [np.zeros((3, 4), np.float32), np.zeros((4, 2), np.float32)]
    c = np.array([0.9, -0.4, 0.05, -2.0], np.float32)
    b = [np.array([0.1, 0.2, -0.3], np.float32), c]
    x = np.array([[1.0, -1.0, 0.5]], np.float32)
    eta, lam, P1, T = 0.3, 0.02, 1.5, 8
    _, _, en = oracle.persample_relax_f64(sizes, "tanh", eta, W, b, [1.0, P1, 1.0], x, T,
                                          act_reg=lam, want_energy=True)
    fc = np.tanh(c.astype(np.float64))
    e0 = 0.5 * np.sum((x[0].astype(np.float64) - np.tanh(b[0].astype(np.float64))) ** 2)
    m = np.zeros(4)
    for t in range(T):
        assert abs(en[t, 0] - (e0 + 0.5 * P1 * np.sum((m - fc) ** 2))) < 1e-12
        m = m - eta * (P1 * (m - fc) + lam * np.sign(m))


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("ffg,act_reg", [(False, 0.0), (True, 0.0), (False, 0.01), (True, 0.003)])
def test_oracle_matches_autograd(oracle, act, ffg, act_reg):
    sizes = [8, 11, 6, 3]
    W, b, _ = make_net(sizes, seed=11, bias_scale=0.2)
    P = [1.0, 0.7, 1.4, 1.0]
    x = make_inputs(5, 8, seed=12)
    T = 9
    top_ref, st_ref, en_ref = autograd_relax(sizes, act, 0.1, W, b, P, x, T, act_reg=act_reg, ffg=ffg)
    top, st, en = oracle.persample_relax_f64(sizes, act, 0.1, W, b, P, x, T, act_reg=act_reg, ffg=ffg,
                                             want_states=True, want_energy=True)
    assert np.max(np.abs(top - top_ref)) < 1e-10
    for l in range(len(sizes)):
        assert np.max(np.abs(st[l] - st_ref[l])) < 1e-10
    assert np.max(np.abs(en - en_ref)) < 1e-10
    # the fp32 batched restatement tracks it at fp32 accuracy
    top32, st32, en32 = oracle.batched_relax(sizes, act, 0.1, W, b, P, x, T, act_reg=act_reg, ffg=ffg,
                                             want_states=True, want_energy=True)
    assert close(top32, top_ref, 1e-5)
    assert close(en32, en_ref, 1e-5)


@pytest.mark.parametrize("act", ACTS)
def test_ffg_start_keeps_the_free_top_exactly_zero(oracle, act):
    # With the FFG warm start every hidden layer starts at f of its prediction
    # from the (zero) layer above, so step 1's errors above layer 0 vanish and
    # the free top's update is exactly zero: the top is 0 after step 1 in both
    # restatements.  On this network it leaves zero at step 2, once lambda
    # sign(M) has moved the layer below off its warm start.
    sizes = [9, 13, 7, 1, 6]
    W, b, P = make_net(sizes, seed=23, bias_scale=0.5)
    x = make_inputs(4, 9, seed=24)
    for T, zero in ((1, True), (2, False)):
        _, st, _ = oracle.persample_relax_f64(sizes, act, 0.08, W, b, P, x, T, act_reg=0.01, ffg=True,
                                              want_states=True)
        _, st32, _ = oracle.batched_relax(sizes, act, 0.08, W, b, P, x, T, act_reg=0.01, ffg=True,
                                          want_states=True)
        assert np.all(st[-1] == 0) == zero and np.all(st32[-1] == 0) == zero


def test_batched_matches_per_sample_reference_tolerance(oracle):
    # BatchedPcForwardTests.cs:44-72 shape: [6,10,4] tanh, eta 0.1, inputs U(-1,1), T=15
    sizes = [6, 10, 4]
    W, b, P = make_net(sizes, seed=0, bias_scale=0.1)
    x = make_inputs(5, 6, seed=3, dist="uniform11")
    top64, _, _ = oracle.persample_relax_f64(sizes, "tanh", 0.1, W, b, P, x, 15)
    top32, _, _ = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, x, 15)
    assert close(top32, top64, 1e-3)   # the reference test's tolerance
    assert close(top32, top64, 1e-5)   # and the fp32 accuracy actually reached


def test_batched_ffg_matches_per_sample(oracle):
    # BatchedPcForwardTests.cs:74-92: FFG on, T=10
    sizes = [6, 10, 4]
    W, b, P = make_net(sizes, seed=1, bias_scale=0.1)
    x = make_inputs(4, 6, seed=5, dist="uniform11")
    top64, _, _ = oracle.persample_relax_f64(sizes, "tanh", 0.1, W, b, P, x, 10, ffg=True)
    top32, _, _ = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, x, 10, ffg=True)
    assert close(top32, top64, 1e-5)


@pytest.mark.parametrize("mode", ["f16", "bf16"])
def test_mixed_tracks_float(oracle, mode):
    # BatchedPcForwardTests.cs:94-111: mixed within 5e-2*(1+|x|) of float
    sizes = [6, 10, 4]
    W, b, P = make_net(sizes, seed=2, bias_scale=0.1)
    x = make_inputs(4, 6, seed=7, dist="uniform11")
    full, _, _ = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, x, 15)
    mixed, _, _ = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, x, 15, round_mode=mode)
    assert close(mixed, full, 5e-2)
    assert not np.array_equal(mixed, full)


def _rel_rms(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)))


@pytest.mark.parametrize("mode", ["bf16", "f16"])
@pytest.mark.parametrize("act", ["tanh", "gelu"])
def test_mixed_rounding_points_against_float64_statement(oracle, mode, act):
    # The oracle's 16-bit relaxation (W and W^T rounded once, the state and
    # delta operands rounded at every GEMM, Gemm.cs:44-60 as BatchedPcForward
    # calls it) against an independent float64 torch statement that rounds the
    # same four operands (tests/autograd_ref.py:mixed_relax_f64).  Rare
    # rounding-boundary flips (fp32 and float64 values on either side of a
    # 16-bit midpoint) keep the two from agreeing bit for bit, so the
    # comparison is the relative RMS of the whole energy trace.  Leaving any
    # one rounding point out of the statement moves it at least 2.5 times
    # further from the oracle than the faithful statement is: every point is
    # pinned.
    from tests.autograd_ref import ROUND_POINTS, mixed_relax_f64
    sizes = [96, 130, 64, 16]
    W, b, P = make_net(sizes, seed=5, init="fanin", bias_scale=0.1)
    x = make_inputs(40, 96, seed=1)
    top, _, en = oracle.batched_relax(sizes, act, 0.05, W, b, P, x, 15, round_mode=mode, want_energy=True)
    ttop, ten = mixed_relax_f64(sizes, act, 0.05, W, b, P, x, 15, mode)
    same = _rel_rms(en, ten)
    assert same < (1e-5 if mode == "bf16" else 5e-6), same
    assert close(top, ttop, 2e-3)
    for point in ROUND_POINTS:
        _, den = mixed_relax_f64(sizes, act, 0.05, W, b, P, x, 15, mode, drop=(point,))
        dropped = _rel_rms(en, den)
        assert dropped > 2.5 * same, (point, dropped, same)


def test_rows_are_independent(oracle):
    sizes = [10, 7, 5]
    W, b, P = make_net(sizes, seed=13)
    x = make_inputs(9, 10, seed=14)
    perm = np.random.default_rng(0).permutation(9)
    top, _, en = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, x, 6, want_energy=True)
    topp, _, enp = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, x[perm], 6, want_energy=True)
    assert np.array_equal(top[perm], topp)
    assert np.array_equal(en[:, perm], enp)


# ------------------------------------------------------------- early exit

def test_exit_disabled_is_fixed_step_bit_for_bit(oracle):
    # AdaptiveInferenceTests.cs:58-72: epsilon = 0 is the fixed-step path exactly
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42, bias_scale=0.1)
    x = np.array([[1, 0, 0, 0], [0, 0, 0, 1]], np.float32)
    top, _, _ = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, x[:1], 20)
    used, fe, topr = oracle.ragged_relax(sizes, "tanh", 0.1, W, b, P, x[:1], [0, 1], [20],
                                         exit_rule="relative", exit_thr=0.0)
    assert used[0] == 20 and np.isfinite(fe[0]) and fe[0] >= 0
    assert np.array_equal(topr, top)


def test_relative_exit_properties(oracle):
    # AdaptiveInferenceTests.cs:97-114: fires, epsilon-monotone, budget-invariant
    sizes = [4, 8, 2]
    W, b, P = make_net(sizes, seed=42, bias_scale=0.1)
    x = np.array([[1, 0, 0, 0]], np.float32)

    def used(budget, eps):
        u, _, _ = oracle.ragged_relax(sizes, "tanh", 0.1, W, b, P, x, [0, 1], [budget],
                                      exit_rule="relative", exit_thr=eps)
        return int(u[0])

    loose, tight, full = used(60, 1e-2), used(60, 1e-4), used(60, 0.0)
    assert loose < 60 and loose <= tight and full == 60
    assert used(200, 1e-2) == loose


def test_relative_exit_step_by_hand(oracle):
    # The exit step is the first t >= 2 with E_{t-1} - E_t < eps * E_{t-1}.
    sizes = [5, 6, 3]
    W, b, P = make_net(sizes, seed=3, bias_scale=0.1)
    x = make_inputs(1, 5, seed=9)
    _, _, en = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, x, 80, want_energy=True)
    e = en[:, 0]
    for eps in (1e-1, 3e-2, 1e-2, 1e-3):
        want = 80
        for t in range(1, 80):
            if np.float32(e[t - 1]) - np.float32(e[t]) < np.float32(eps) * max(np.float32(e[t - 1]), np.float32(1e-12)):
                want = t + 1
                break
        u, fe, _ = oracle.ragged_relax(sizes, "tanh", 0.1, W, b, P, x, [0, 1], [80],
                                       exit_rule="relative", exit_thr=eps)
        assert int(u[0]) == want
        assert abs(fe[0] - e[want - 1]) <= 1e-6 * (1 + abs(e[want - 1]))


def test_absolute_exit_and_ragged_equals_separate_batches(oracle):
    sizes = [6, 5, 3]
    W, b, P = make_net(sizes, seed=21)
    x = make_inputs(7, 6, seed=22) * 0.1
    offs = [0, 1, 4, 7]
    steps = [30, 12, 40]
    u, fe, top = oracle.ragged_relax(sizes, "tanh", 0.1, W, b, P, x, offs, steps,
                                     exit_rule="absolute", exit_thr=1e-3)
    for r in range(3):
        xr = x[offs[r]:offs[r + 1]]
        _, _, en = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, xr, steps[r], want_energy=True)
        per = en.sum(axis=1) / len(xr)
        hit = np.nonzero(per < 1e-3)[0]
        want = int(hit[0]) + 1 if hit.size else steps[r]
        assert int(u[r]) == want
        t_r, _, _ = oracle.batched_relax(sizes, "tanh", 0.1, W, b, P, xr, want)
        assert np.array_equal(top[offs[r]:offs[r + 1]], t_r)
