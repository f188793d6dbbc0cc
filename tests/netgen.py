"""Seeded synthetic networks and inputs shared by the tests (numpy only).

Weights follow the reference's initialisers: Xavier-normal
sigma = sqrt(2 / (fan_in + fan_out)) with fan_in = s_l, fan_out = s_{l-1}
(RandomUtils.cs:63-67 via Layer.cs:174), or N(0, 1/fan_in) for the GELU
configurations; biases are zero (RandomUtils.cs:104) unless a test asks for
random ones.
"""
import numpy as np


def make_net(sizes, seed=0, init="xavier", bias_scale=0.0, precisions=None):
    rng = np.random.default_rng(seed)
    W, b = [], []
    for l in range(1, len(sizes)):
        lo, sz = sizes[l - 1], sizes[l]
        if init == "xavier":
            std = np.sqrt(2.0 / (sz + lo))
        elif init == "fanin":
            std = np.sqrt(1.0 / sz)
        else:
            std = float(init)
        W.append((rng.standard_normal((lo, sz)) * std).astype(np.float32))
        b.append((rng.standard_normal(lo) * bias_scale).astype(np.float32))
    if precisions is None:
        precisions = np.ones(len(sizes), dtype=np.float32)
    return W, b, np.asarray(precisions, dtype=np.float32)


def make_inputs(batch, size, seed=1, dist="normal"):
    rng = np.random.default_rng(seed)
    if dist == "normal":
        return rng.standard_normal((batch, size)).astype(np.float32)
    if dist == "uniform01":
        return rng.random((batch, size)).astype(np.float32)
    if dist == "uniform11":
        return (rng.random((batch, size)) * 2 - 1).astype(np.float32)
    raise ValueError(dist)


def _rel(a, b):
    """Elementwise |a-b| / (1+|b|), with equal values (infinities of one sign,
    NaN against NaN) at 0 and a NaN or an infinity on one side only at inf, so
    a diverging network compares by where it overflowed and no NaN reaches a
    reduction (Python's max() skips a NaN that is not its first argument)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    same = (a == b) | (np.isnan(a) & np.isnan(b))
    with np.errstate(invalid="ignore"):
        d = np.abs(a - b) / (1.0 + np.abs(b))
    return np.where(same, 0.0, np.where(np.isnan(d), np.inf, d))


def close(a, b, tol):
    """The reference tests' element bound |a-b| <= tol*(1+|b|) (BatchedPcForwardTests.cs:67)."""
    return bool(np.all(_rel(a, b) <= tol))


def max_rel(a, b):
    d = _rel(a, b)
    return float(np.max(d)) if d.size else 0.0
