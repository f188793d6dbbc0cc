"""Seeded random networks through the settling entry points, against the oracle.

Each case draws its layer count (2 to 6), its widths around the tile and
padding boundaries (1 to 330 wide: 63/64/65, 127/128/129, 255/256/257), its
batch (1 to 257 rows), the activation, the operand type, the FFG sweep,
activity regularisation, non-unit precisions, eta and the step count, so the
combinations the hand-written cases do not name get settled too.  Every case
is small enough for the oracle to finish in well under a second.

Bounds, as in the other parity tests (|a-b| <= tol (1+|b|),
BatchedPcForwardTests.cs:67): 1e-4 for fp32; 2e-3 for 16-bit operands against
the oracle run with the same operand rounding.
"""
import numpy as np
import pytest

from predicitivecoding_amd import PcDeviceModel
from tests.gpu_util import ACT_ID, ROUND, build_case, run_gpu, run_oracle
from tests.netgen import make_inputs, max_rel

pytestmark = pytest.mark.gpu

WIDTHS = [1, 2, 5, 31, 63, 64, 65, 100, 127, 128, 129, 200, 255, 256, 257, 330]
ROWS = [1, 2, 7, 63, 64, 65, 129, 257]
ACTS = sorted(ACT_ID)
TOL = {"f32": 1e-4, "bf16": 2e-3, "f16": 2e-3}


def draw(seed, top_width=None, dtypes=("f32", "f32", "bf16", "f16")):
    rng = np.random.default_rng(1000 + seed)
    L = int(rng.integers(2, 7))
    sizes = [int(rng.choice(WIDTHS)) for _ in range(L)]
    if top_width is not None:
        sizes[-1] = int(rng.integers(*top_width))
    return dict(
        sizes=sizes,
        act=str(rng.choice(ACTS)),
        dtype=str(rng.choice(dtypes)),
        ffg=bool(rng.random() < 0.3),
        act_reg=0.01 if rng.random() < 0.3 else 0.0,
        precisions=[float(v) for v in rng.uniform(0.5, 1.5, L)] if rng.random() < 0.4 else None,
        eta=float(rng.uniform(0.02, 0.15)),
        batch=int(rng.choice(ROWS)),
        steps=int(rng.integers(1, 9)),
        bias_scale=float(rng.choice([0.0, 0.2])),
        init=str(rng.choice(["xavier", "fanin"])),
    )


def case_of(c, seed):
    return build_case(c["sizes"], c["act"], c["eta"], act_reg=c["act_reg"], ffg=c["ffg"], seed=seed, init=c["init"],
                      bias_scale=c["bias_scale"], precisions=c["precisions"], batch=c["batch"], xseed=seed + 7)


def describe(c):
    return (f"sizes={c['sizes']} {c['act']} {c['dtype']} ffg={c['ffg']} act_reg={c['act_reg']} "
            f"prec={'yes' if c['precisions'] else 'no'} eta={c['eta']:.3f} B={c['batch']} T={c['steps']}")


@pytest.mark.parametrize("seed", range(24))
def test_random_relax(oracle, seed):
    c = draw(seed)
    print(describe(c), flush=True)
    snap, W, b, P, x = case_of(c, seed)
    top, st, en = run_gpu(snap, x, c["steps"], dtype=c["dtype"], states=True, energy=True)
    rtop, rst, ren = run_oracle(oracle, snap, W, b, P, x, c["steps"], dtype=c["dtype"], states=True, energy=True)
    errs = dict(top=max_rel(top, rtop), energy=max_rel(en, ren),
                states=max(max_rel(a, r) for a, r in zip(st, rst)))
    print(" ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert np.array_equal(st[0], x), "the input layer stays clamped"
    assert all(v < TOL[c["dtype"]] for v in errs.values()), errs


@pytest.mark.parametrize("seed", range(8))
def test_random_ragged(oracle, seed):
    # fp32, so the exit steps compare exactly: the relative rule at a random
    # epsilon, the absolute rule at a threshold inside the requests' energy range
    c = draw(100 + seed, dtypes=("f32",))
    rng = np.random.default_rng(2000 + seed)
    R = int(rng.integers(1, 7))
    rows = [int(rng.choice([1, 2, 5, 17, 64, 65])) for _ in range(R)]
    offs = np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)
    steps = rng.integers(1, 10, size=R).astype(np.int32)
    snap, W, b, P, _ = case_of(c, 100 + seed)
    x = make_inputs(int(offs[-1]), c["sizes"][0], seed=seed + 11)
    act = c["act"]
    rule = ["none", "relative", "absolute"][seed % 3]
    thr = 0.0
    if rule == "relative":
        thr = float(rng.uniform(0.02, 0.3))
    elif rule == "absolute":
        _, fe, _ = oracle.ragged_relax(c["sizes"], act, c["eta"], W, b, P, x, offs, steps, act_reg=c["act_reg"],
                                       ffg=c["ffg"])
        per = fe / np.diff(offs)
        thr = float(np.median(per)) * 1.013 if np.all(np.isfinite(per)) else 1.0
    print(describe(c), f"R={R} rows={rows} steps={steps.tolist()} rule={rule} thr={thr:.3g}", flush=True)
    m = PcDeviceModel(snap, "f32")
    try:
        used, fe, top = m.relax_ragged(x, offs, steps, rule, thr)
    finally:
        m.close()
    rused, rfe, rtop = oracle.ragged_relax(c["sizes"], act, c["eta"], W, b, P, x, offs, steps, exit_rule=rule,
                                           exit_thr=thr, act_reg=c["act_reg"], ffg=c["ffg"])
    print("used", used.tolist(), "oracle", rused.tolist(), flush=True)
    assert np.array_equal(used, rused)
    errs = dict(top=max_rel(top, rtop), energy=max_rel(fe, rfe))
    assert all(v < 1e-4 for v in errs.values()), errs


@pytest.mark.parametrize("seed", range(8))
def test_random_classify(oracle, seed):
    c = draw(200 + seed, top_width=(2, 13))
    print(describe(c), flush=True)
    snap, W, b, P, x = case_of(c, 200 + seed)
    m = PcDeviceModel(snap, c["dtype"])
    try:
        ce, cls, be = m.classify(x, c["steps"])
    finally:
        m.close()
    rce, rcls, rbe = oracle.classify(c["sizes"], c["act"], c["eta"], W, b, P, x, c["steps"], act_reg=c["act_reg"],
                                     ffg=c["ffg"], round_mode=ROUND[c["dtype"]])
    tol = TOL[c["dtype"]]
    errs = dict(class_energies=max_rel(ce, rce), best_energy=max_rel(be, rbe))
    print(" ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v < tol for v in errs.values()), errs
    # the chosen class is the oracle's wherever the two lowest energies are
    # further apart than the bound
    srt = np.sort(rce.astype(np.float64), axis=1)
    margin = srt[:, 1] - srt[:, 0] if rce.shape[1] > 1 else np.full(len(rcls), np.inf)
    decided = margin > 2 * tol * (1 + np.abs(srt[:, 0]))
    assert np.array_equal(cls[decided], rcls[decided])


@pytest.mark.parametrize("seed", range(6))
def test_random_learn(oracle, seed):
    c = draw(300 + seed, dtypes=("f32",))
    print(describe(c), flush=True)
    snap, W, b, P, x = case_of(c, 300 + seed)
    rng = np.random.default_rng(3000 + seed)
    y = rng.standard_normal((c["batch"], c["sizes"][-1])).astype(np.float32)
    eta_w = float(rng.uniform(0.005, 0.05))
    wd = float(rng.choice([0.0, 1e-3]))
    m = PcDeviceModel(snap, "f32")
    try:
        en = m.learn(x, y, c["steps"], eta_w, wd)
        gw, gb = m.get_weights()
    finally:
        m.close()
    rw, rb, ren = oracle.learn(c["sizes"], c["act"], c["eta"], W, b, P, x, y, c["steps"], eta_w, weight_decay=wd,
                               act_reg=c["act_reg"], ffg=c["ffg"])
    errs = dict(weights=max(max_rel(a, r) for a, r in zip(gw, rw)), biases=max(max_rel(a, r) for a, r in zip(gb, rb)),
                energy=max_rel(en, ren))
    print(" ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v < 1e-4 for v in errs.values()), errs


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_deep_network_spans_several_launches(oracle, dtype):
    # 21 levels: each phase has 20 problems, more than one grouped launch holds
    # (16), so every phase runs as two launches; relax, classify, the ragged
    # path with an exit and (fp32) the learning step all go through them
    rng = np.random.default_rng(77)
    sizes = [int(v) for v in rng.choice([16, 33, 64, 70], size=21)]
    sizes[-1] = 5
    snap, W, b, P, x = build_case(sizes, "tanh", 0.05, seed=77, init="fanin", bias_scale=0.1, batch=70)
    tol = TOL[dtype]
    top, st, en = run_gpu(snap, x, 6, dtype=dtype, states=True, energy=True)
    rtop, rst, ren = run_oracle(oracle, snap, W, b, P, x, 6, dtype=dtype, states=True, energy=True)
    errs = dict(top=max_rel(top, rtop), energy=max_rel(en, ren), states=max(max_rel(a, r) for a, r in zip(st, rst)))
    print("relax", " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v < tol for v in errs.values()), errs
    m = PcDeviceModel(snap, dtype)
    try:
        ce, cls, be = m.classify(x[:9], 4)
        offs = np.array([0, 3, 40, 70], np.int32)
        steps = np.array([5, 9, 2], np.int32)
        used, fe, rtop2 = m.relax_ragged(x, offs, steps, "relative", 0.05) if dtype == "f32" else (None, None, None)
    finally:
        m.close()
    rce, rcls, _ = oracle.classify(sizes, "tanh", 0.05, W, b, P, x[:9], 4, round_mode=ROUND[dtype])
    assert max_rel(ce, rce) < tol
    if dtype == "f32":
        rused, rfe, rrtop = oracle.ragged_relax(sizes, "tanh", 0.05, W, b, P, x, offs, steps, exit_rule="relative",
                                                exit_thr=0.05)
        print("used", used.tolist(), "oracle", rused.tolist(), flush=True)
        assert np.array_equal(used, rused)
        assert max_rel(fe, rfe) < tol and max_rel(rtop2, rrtop) < tol
        y = np.eye(5, dtype=np.float32)[np.arange(70) % 5]
        m = PcDeviceModel(snap, "f32")
        try:
            en_learn = m.learn(x, y, 4, 0.02)
            gw, gb = m.get_weights()
        finally:
            m.close()
        rw, rb, ren2 = oracle.learn(sizes, "tanh", 0.05, W, b, P, x, y, 4, 0.02)
        assert max(max_rel(a, r) for a, r in zip(gw, rw)) < 1e-4
        assert max(max_rel(a, r) for a, r in zip(gb, rb)) < 1e-4
        assert max_rel(en_learn, ren2) < 1e-4


OPTION_SETS = [
    {},
    {"tile_order": 1},
    {"split_min": 2},
    {"split_min": 40},
    {"split_k": 0},
    {"use_graph": 0},
    {"k_stagger": 0},
    {"profile": 1},
    {"tile_order": 1, "split_min": 2, "use_graph": 0, "k_stagger": 5},
    {"tile": 32},
    {"tile": 32, "split_min": 2},
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("opts", OPTION_SETS, ids=lambda o: "-".join(f"{k}{v}" for k, v in o.items()) or "defaults")
def test_relaxation_options_keep_parity(oracle, dtype, opts):
    # a 64-row batch on a network with a long K sweep, so the split-K paths and
    # several problems per phase are in play; every option combination settles
    # to the oracle's result
    snap, W, b, P, x = build_case([300, 1030, 260, 70], "gelu", 0.08, batch=64, seed=41, init="fanin",
                                  bias_scale=0.1)
    m = PcDeviceModel(snap, dtype)
    try:
        for k, v in opts.items():
            m.set_option(k, v)
        top, st, en = m.relax(x, 7, want_states=True, want_energy=True)
        prof = m.profile_result() if opts.get("profile") else None
    finally:
        m.close()
    rtop, rst, ren = run_oracle(oracle, snap, W, b, P, x, 7, dtype=dtype, states=True, energy=True)
    errs = dict(top=max_rel(top, rtop), energy=max_rel(en, ren), states=max(max_rel(a, r) for a, r in zip(st, rst)))
    print(opts, " ".join(f"{k}={v:.2e}" for k, v in errs.items()), prof, flush=True)
    assert all(v < TOL[dtype] for v in errs.values()), errs
    if prof is not None:
        err_ms, upd_ms, launches = prof
        assert launches == 7 and err_ms > 0 and upd_ms > 0
