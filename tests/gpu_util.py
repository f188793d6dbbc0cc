"""Helpers for the GPU parity tests (which call the library through its C ABI)."""
import numpy as np

from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel
from tests.netgen import make_inputs, make_net

ACT_ID = {"linear": 0, "tanh": 1, "relu": 2, "sigmoid": 3, "gelu": 4}
ROUND = {"f32": "none", "bf16": "bf16", "f16": "f16"}


def build_case(sizes, act="tanh", eta=0.1, act_reg=0.0, ffg=False, seed=0, init="xavier", bias_scale=0.0,
               precisions=None, batch=8, xdist="normal", xseed=1):
    W, b, P = make_net(sizes, seed=seed, init=init, bias_scale=bias_scale, precisions=precisions)
    x = make_inputs(batch, sizes[0], seed=xseed, dist=xdist)
    snap = GenerativeSnapshot(sizes, ACT_ID[act], eta, act_reg, ffg, W, b, list(P))
    return snap, W, b, P, x


def run_gpu(snap, x, steps, dtype="f32", states=False, energy=False, options=None):
    m = PcDeviceModel(snap, dtype)
    try:
        for k, v in (options or {}).items():
            m.set_option(k, v)
        return m.relax(x, steps, want_states=states, want_energy=energy)
    finally:
        m.close()


def run_oracle(oracle, snap, W, b, P, x, steps, dtype="f32", states=False, energy=False):
    act = [k for k, v in ACT_ID.items() if v == int(snap.activation)][0]
    return oracle.batched_relax(snap.layer_sizes, act, snap.state_learning_rate, W, b, P, x, steps,
                                act_reg=snap.activity_regularization, ffg=snap.use_feedforward_gist_init,
                                round_mode=ROUND[dtype], want_states=states, want_energy=energy)
