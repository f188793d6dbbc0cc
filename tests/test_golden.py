"""The committed golden fixtures (tests/golden/*.npz, float64 autograd of the
free energy) against the CPU oracle: the float64 per-sample restatement to
1e-10, the fp32 batched restatement to fp32 accuracy."""
import numpy as np
import pytest

from tests.golden.make_golden import fixtures, load
from tests.netgen import close

FIXTURES = fixtures()


def test_fixtures_present():
    assert len(FIXTURES) >= 8


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: p.rsplit("/", 1)[-1][:-4])
def test_oracle_reproduces_golden(oracle, path):
    g = load(path)
    kw = dict(act_reg=g["act_reg"], ffg=g["ffg"], want_states=True, want_energy=True)
    top, st, en = oracle.persample_relax_f64(g["sizes"], g["act"], g["eta"], g["W"], g["b"], g["precisions"],
                                             g["x"], g["steps"], **kw)
    assert np.max(np.abs(top - g["top"])) < 1e-10
    assert np.max(np.abs(en - g["energy"])) < 1e-10
    for a, r in zip(st, g["states"]):
        assert np.max(np.abs(a - r)) < 1e-10
    top32, _, en32 = oracle.batched_relax(g["sizes"], g["act"], g["eta"], g["W"], g["b"], g["precisions"],
                                          g["x"], g["steps"], **kw)
    assert close(top32, g["top"], 1e-5) and close(en32, g["energy"], 1e-5)
