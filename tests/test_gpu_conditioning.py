"""Ill-conditioned networks: where fp32 itself cannot hold the 1e-4 bound.

Random-network sweeps put about 1% of networks outside |a-b| <= 1e-4 (1+|b|)
against the fp32 oracle.  Most of them are ill-conditioned: linear networks
whose states grow by orders of magnitude over the steps (a narrow hidden layer
with a large gain), on which the fp32 oracle is itself as far from the float64
per-sample settling (Network.InferGetTop in double precision, the oracle's
pco_persample_relax_f64) as the GPU is from the fp32 oracle.  These cases pin
that explanation: each network is chosen so that the fp32 oracle misses
float64 by more than 1e-4 (the premise), and the GPU's result must then be as
close to float64 as the fp32 oracle's is (within a factor 10), i.e. no worse
than fp32 arithmetic allows on that network.
"""
import numpy as np
import pytest

from tests.gpu_util import build_case, run_gpu
from tests.netgen import max_rel

pytestmark = pytest.mark.gpu

# (seed, weight standard deviation): [40, 2, 33, 8] linear networks, eta 0.1,
# 16 inputs, 8 steps; the fp32 oracle's error against float64 is 1.1e-3,
# 8.1e-4, 3.6e-4 and 3.5e-4 (states reaching 2.7e5 to 1.5e7)
CASES = [(15, 1.5), (27, 2.0), (21, 2.0), (11, 2.0)]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_gpu_is_within_the_fp32_envelope_on_ill_conditioned_networks(oracle, case):
    seed, std = CASES[case]
    sizes = [40, 2, 33, 8]
    snap, W, b, P, x = build_case(sizes, "linear", 0.1, batch=16, seed=seed, init=std, xseed=seed + 1)
    top, _, en = run_gpu(snap, x, 8, energy=True)
    t32, _, e32 = oracle.batched_relax(sizes, "linear", 0.1, W, b, P, x, 8, want_energy=True)
    t64, _, e64 = oracle.persample_relax_f64(sizes, "linear", 0.1, W, b, P, x, 8, want_energy=True)
    err32 = max(max_rel(t32, t64), max_rel(e32, e64))
    err_gpu = max(max_rel(top, t64), max_rel(en, e64))
    print(f"seed {seed} std {std}: |states| up to {np.abs(t64).max():.1e}; fp32 oracle vs float64 {err32:.2e}, "
          f"GPU vs float64 {err_gpu:.2e}, GPU vs fp32 oracle {max(max_rel(top, t32), max_rel(en, e32)):.2e}",
          flush=True)
    assert err32 > 1e-4, "the premise: fp32 arithmetic itself misses float64 by more than the bound here"
    assert err_gpu <= 10 * err32
