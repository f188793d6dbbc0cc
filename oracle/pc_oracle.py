"""ctypes binding of ``libpcoracle.so`` (the C restatement in ``pc_oracle.c``).

Test infrastructure only: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py.  Every function mirrors a reference
routine cited in ``pc_oracle.c``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libpcoracle.so")
_lib = None

ACT = {"linear": 0, "tanh": 1, "relu": 2, "sigmoid": 3, "gelu": 4}
ROUND = {"none": 0, "f16": 1, "bf16": 2}
EXIT = {"none": 0, "relative": 1, "absolute": 2}

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p


def build() -> str:
    """Compile the oracle with its Makefile; returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.pco_act_apply_f32.argtypes = [ctypes.c_int, _f32p, _f32p, ctypes.c_long]
        L.pco_act_deriv_f32.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p, ctypes.c_long]
        L.pco_act_apply_f64.argtypes = [ctypes.c_int, _f64p, _f64p, ctypes.c_long]
        L.pco_act_deriv_f64.argtypes = [ctypes.c_int, _f64p, _f64p, _f64p, ctypes.c_long]
        L.pco_round.argtypes = [ctypes.c_int, _f32p, _f32p, ctypes.c_long]
        L.pco_bf16_bits.argtypes = [_f32p, _u16p, ctypes.c_long]
        L.pco_gemm.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int, _f32p, ctypes.c_int]
        L.pco_set_threads.argtypes = [ctypes.c_int]
        L.pco_get_threads.restype = ctypes.c_int
        L.pco_batched_relax.argtypes = [
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
            _f32p, _f32p, _f32p, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, _f32p, _vp, _vp]
        L.pco_batched_relax.restype = ctypes.c_int
        L.pco_ragged_relax.argtypes = [
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
            _f32p, _f32p, _f32p, ctypes.c_int, _f32p, _i32p, _i32p, ctypes.c_int,
            ctypes.c_int, ctypes.c_float, _i32p, _f32p, _f32p]
        L.pco_ragged_relax.restype = ctypes.c_int
        L.pco_persample_relax_f64.argtypes = [
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_int,
            _f64p, _f64p, _f64p, _f64p, _vp, ctypes.c_int, ctypes.c_int, _f64p, _vp, _vp]
        L.pco_persample_relax_f64.restype = ctypes.c_int
        L.pco_clamped_relax.argtypes = [
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
            _f32p, _f32p, _f32p, ctypes.c_int, _f32p, _f32p, ctypes.c_int, ctypes.c_int, _vp, _vp]
        L.pco_clamped_relax.restype = ctypes.c_int
        L.pco_classify.argtypes = [
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
            _f32p, _f32p, _f32p, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, _f32p, _i32p, _f32p]
        L.pco_classify.restype = ctypes.c_int
        L.pco_classify_adaptive.argtypes = [
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
            _f32p, _f32p, _f32p, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
            _f32p, _i32p, _i32p, _f32p, _i32p]
        L.pco_classify_adaptive.restype = ctypes.c_int
        L.pco_learn.argtypes = [
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
            _f32p, _f32p, _f32p, ctypes.c_int, _f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
            ctypes.c_float, _vp, _vp, _vp]
        L.pco_learn.restype = ctypes.c_int
        _lib = L
    return _lib


def set_threads(n: int) -> None:
    lib().pco_set_threads(int(n))


def get_threads() -> int:
    return int(lib().pco_get_threads())


def act_apply(act: str, x, dtype=np.float32):
    x = np.ascontiguousarray(x, dtype=dtype)
    y = np.empty_like(x)
    fn = lib().pco_act_apply_f32 if dtype == np.float32 else lib().pco_act_apply_f64
    fn(ACT[act], x.ravel(), y.ravel(), x.size)
    return y


def act_deriv(act: str, pre, dtype=np.float32):
    pre = np.ascontiguousarray(pre, dtype=dtype)
    y = act_apply(act, pre, dtype)
    d = np.empty_like(pre)
    fn = lib().pco_act_deriv_f32 if dtype == np.float32 else lib().pco_act_deriv_f64
    fn(ACT[act], pre.ravel(), y.ravel(), d.ravel(), pre.size)
    return d


def round16(mode: str, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().pco_round(ROUND[mode], x.ravel(), y.ravel(), x.size)
    return y


def bf16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = np.empty(x.shape, dtype=np.uint16)
    lib().pco_bf16_bits(x.ravel(), b.ravel(), x.size)
    return b


def gemm(a, b, round_mode: str = "none"):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), dtype=np.float32)
    lib().pco_gemm(a.ravel(), m, k, b.ravel(), n, c.ravel(), ROUND[round_mode])
    return c


def _flat(arrs, dtype):
    if not arrs:
        return np.zeros(1, dtype=dtype)
    return np.ascontiguousarray(np.concatenate([np.asarray(a, dtype=dtype).ravel() for a in arrs]))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def batched_relax(sizes, act, eta, weights, biases, precisions, x0, steps,
                  act_reg=0.0, ffg=False, round_mode="none", want_states=False, want_energy=False):
    """BatchedPcForward.InferGetTopBatch in fp32 (optionally with 16-bit operand
    rounding).  Returns (top [B,s_top], states list or None, energy [T,B] or None)."""
    sizes = np.ascontiguousarray(sizes, dtype=np.int32)
    x0 = np.ascontiguousarray(x0, dtype=np.float32)
    B = x0.shape[0]
    top = np.empty((B, int(sizes[-1])), dtype=np.float32)
    states = np.empty(B * int(sizes.sum()), dtype=np.float32) if want_states else None
    energy = np.empty((steps, B), dtype=np.float32) if want_energy else None
    rc = lib().pco_batched_relax(sizes, len(sizes), ACT[act], eta, act_reg, int(ffg),
                                 _flat(weights, np.float32), _flat(biases, np.float32),
                                 np.ascontiguousarray(precisions, dtype=np.float32), ROUND[round_mode],
                                 x0.ravel(), B, int(steps), top.ravel(), _ptr(states), _ptr(energy))
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    st = None
    if want_states:
        st, off = [], 0
        for s in sizes:
            st.append(states[off:off + B * int(s)].reshape(B, int(s)))
            off += B * int(s)
    return top, st, energy


def persample_relax_f64(sizes, act, eta, weights, biases, precisions, x0, steps,
                        act_reg=0.0, ffg=False, want_states=False, want_energy=False, top_clamp=None):
    """Network.InferGetTop(x, steps, resetState: true) per sample, in float64;
    with top_clamp [B, s_top] the top layer is held there (InferCore with a label)."""
    sizes = np.ascontiguousarray(sizes, dtype=np.int32)
    x0 = np.ascontiguousarray(x0, dtype=np.float64)
    B = x0.shape[0]
    tc = None if top_clamp is None else np.ascontiguousarray(top_clamp, dtype=np.float64).reshape(B, int(sizes[-1]))
    top = np.empty((B, int(sizes[-1])), dtype=np.float64)
    states = np.empty(B * int(sizes.sum()), dtype=np.float64) if want_states else None
    energy = np.empty((steps, B), dtype=np.float64) if want_energy else None
    rc = lib().pco_persample_relax_f64(sizes, len(sizes), ACT[act], eta, act_reg, int(ffg),
                                       _flat(weights, np.float64), _flat(biases, np.float64),
                                       np.ascontiguousarray(precisions, dtype=np.float64),
                                       x0.ravel(), _ptr(tc), B, int(steps), top.ravel(), _ptr(states),
                                       _ptr(energy))
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    st = None
    if want_states:
        st, off = [], 0
        for s in sizes:
            st.append(states[off:off + B * int(s)].reshape(B, int(s)))
            off += B * int(s)
    return top, st, energy


def ragged_relax(sizes, act, eta, weights, biases, precisions, x0_packed, row_offsets, steps,
                 exit_rule="none", exit_thr=0.0, act_reg=0.0, ffg=False, round_mode="none"):
    """Per-request settling with early exit; returns (steps_used, final_energy, top)."""
    sizes = np.ascontiguousarray(sizes, dtype=np.int32)
    x0 = np.ascontiguousarray(x0_packed, dtype=np.float32)
    offs = np.ascontiguousarray(row_offsets, dtype=np.int32)
    st = np.ascontiguousarray(steps, dtype=np.int32)
    R = len(st)
    used = np.zeros(R, dtype=np.int32)
    fe = np.zeros(R, dtype=np.float32)
    top = np.zeros((x0.shape[0], int(sizes[-1])), dtype=np.float32)
    rc = lib().pco_ragged_relax(sizes, len(sizes), ACT[act], eta, act_reg, int(ffg),
                                _flat(weights, np.float32), _flat(biases, np.float32),
                                np.ascontiguousarray(precisions, dtype=np.float32), ROUND[round_mode],
                                x0.ravel(), offs, st, R, EXIT[exit_rule], exit_thr, used, fe, top.ravel())
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return used, fe, top


def _split_states(states, sizes, B):
    st, off = [], 0
    for sz in sizes:
        st.append(states[off:off + B * int(sz)].reshape(B, int(sz)))
        off += B * int(sz)
    return st


def clamped_relax(sizes, act, eta, weights, biases, precisions, x0, top, steps,
                  act_reg=0.0, ffg=False, round_mode="none"):
    """InferCore with input and top clamped (Network.cs:75-111, clampTop).
    Returns (states list, energy [T, B])."""
    sizes = np.ascontiguousarray(sizes, dtype=np.int32)
    x0 = np.ascontiguousarray(x0, dtype=np.float32)
    B = x0.shape[0]
    top = np.ascontiguousarray(top, dtype=np.float32).reshape(B, int(sizes[-1]))
    states = np.empty(B * int(sizes.sum()), dtype=np.float32)
    energy = np.empty((steps, B), dtype=np.float32)
    rc = lib().pco_clamped_relax(sizes, len(sizes), ACT[act], eta, act_reg, int(ffg),
                                 _flat(weights, np.float32), _flat(biases, np.float32),
                                 np.ascontiguousarray(precisions, dtype=np.float32), ROUND[round_mode],
                                 x0.ravel(), top.ravel(), B, int(steps), _ptr(states), _ptr(energy))
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return _split_states(states, sizes, B), energy


def classify(sizes, act, eta, weights, biases, precisions, x0, steps, act_reg=0.0, ffg=False, round_mode="none"):
    """Network.PredictCore / ClassEnergies per sample: returns
    (class_energies [B, C], best_class [B], best_energy [B])."""
    sizes = np.ascontiguousarray(sizes, dtype=np.int32)
    x0 = np.ascontiguousarray(x0, dtype=np.float32)
    B, C = x0.shape[0], int(sizes[-1])
    ce = np.empty((B, C), dtype=np.float32)
    bc = np.empty(B, dtype=np.int32)
    be = np.empty(B, dtype=np.float32)
    rc = lib().pco_classify(sizes, len(sizes), ACT[act], eta, act_reg, int(ffg),
                            _flat(weights, np.float32), _flat(biases, np.float32),
                            np.ascontiguousarray(precisions, dtype=np.float32), ROUND[round_mode],
                            x0.ravel(), B, int(steps), ce.ravel(), bc, be)
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return ce, bc, be


def classify_adaptive(sizes, act, eta, weights, biases, precisions, x0, max_steps, epsilon, act_reg=0.0,
                      ffg=False, round_mode="none"):
    """Network.PredictAdaptive per sample: returns (class_energies [B, C],
    class_steps [B, C], best_class [B], best_energy [B], steps_used [B])."""
    sizes = np.ascontiguousarray(sizes, dtype=np.int32)
    x0 = np.ascontiguousarray(x0, dtype=np.float32)
    B, C = x0.shape[0], int(sizes[-1])
    ce = np.empty((B, C), dtype=np.float32)
    cs = np.empty((B, C), dtype=np.int32)
    bc = np.empty(B, dtype=np.int32)
    be = np.empty(B, dtype=np.float32)
    su = np.empty(B, dtype=np.int32)
    rc = lib().pco_classify_adaptive(sizes, len(sizes), ACT[act], eta, act_reg, int(ffg),
                                     _flat(weights, np.float32), _flat(biases, np.float32),
                                     np.ascontiguousarray(precisions, dtype=np.float32), ROUND[round_mode],
                                     x0.ravel(), B, int(max_steps), float(epsilon), ce.ravel(), cs.ravel(), bc, be,
                                     su)
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return ce, cs, bc, be, su


# EffortPresets.For (Networks/EffortLevel.cs:33-39): (maxSteps, epsilon) per effort level
EFFORT_PRESETS = {"low": (10, 1e-3), "medium": (30, 1e-4), "high": (100, 1e-5)}


def learn(sizes, act, eta, weights, biases, precisions, x0, labels, steps, eta_w, weight_decay=0.0,
          act_reg=0.0, ffg=False, round_mode="none", hidden=None, want_hidden=False):
    """Network.Learn on a batch (B = 1 is the reference call; B > 1 sums the
    per-sample updates at the pre-call weights); with a 16-bit round_mode,
    LearnMixed on fp32 masters.  `hidden` (a list of [B x s_l] arrays for
    l = 1..L-2, or None for zeros) is the hidden state the settling starts
    from, as the network persisted it.  Returns (new weights, new biases,
    energy [B]), plus the settled hidden states with want_hidden."""
    sizes = np.ascontiguousarray(sizes, dtype=np.int32)
    x0 = np.ascontiguousarray(x0, dtype=np.float32)
    B = x0.shape[0]
    labels = np.ascontiguousarray(labels, dtype=np.float32).reshape(B, int(sizes[-1]))
    W = _flat(weights, np.float32).copy()
    b = _flat(biases, np.float32).copy()
    energy = np.empty(B, dtype=np.float32)
    nh = B * int(sizes[1:-1].sum())
    h_in = None if hidden is None else np.concatenate([np.ascontiguousarray(h, np.float32).ravel() for h in hidden])
    if h_in is not None and h_in.size != nh:
        raise ValueError("hidden must hold the hidden layers' [B x s_l] states")
    h_out = np.empty(max(nh, 1), dtype=np.float32)
    rc = lib().pco_learn(sizes, len(sizes), ACT[act], eta, act_reg, int(ffg), W, b,
                         np.ascontiguousarray(precisions, dtype=np.float32), ROUND[round_mode], x0.ravel(),
                         labels.ravel(),
                         B, int(steps), float(eta_w), float(weight_decay), _ptr(energy),
                         _ptr(h_in) if h_in is not None and nh else None, _ptr(h_out))
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    new_w, new_b, wo, bo = [], [], 0, 0
    for l in range(1, len(sizes)):
        lo, sz = int(sizes[l - 1]), int(sizes[l])
        new_w.append(W[wo:wo + lo * sz].reshape(lo, sz))
        new_b.append(b[bo:bo + lo])
        wo += lo * sz
        bo += lo
    if not want_hidden:
        return new_w, new_b, energy
    out, off = [], 0
    for l in range(1, len(sizes) - 1):
        out.append(h_out[off:off + B * int(sizes[l])].reshape(B, int(sizes[l])))
        off += B * int(sizes[l])
    return new_w, new_b, energy, out
