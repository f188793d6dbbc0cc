"""pcd_pc_relax_noalloc, the allocation-free variant of pcd_pc_relax.

It runs the same kernels with its scratch carved from a library-owned device
array instead of the (model, stream) workspace, so its top states, all states
and per-step energies must equal pcd_pc_relax's bit for bit.  Each case makes
two calls in a row, the second with a smaller batch, after a call of another
model has left its own values in the shared array (stale scratch must not
leak into a result).  A batch whose scratch exceeds the array is refused
before anything is launched.
"""
import numpy as np
import pytest

from tests.netgen import make_inputs, make_net

pytestmark = pytest.mark.gpu

CASES = [
    # sizes, activation id, dtype, ffg, eta, batches (second smaller)
    ([784, 256, 256, 10], 1, "f32", 0, 0.1, (64, 20)),
    ([512, 1024, 256, 32], 4, "bf16", 0, 0.05, (300, 77)),
    ([96, 200, 130, 7], 1, "f32", 1, 0.1, (129, 5)),
    ([256, 512, 64], 3, "f16", 0, 0.1, (40, 3)),
]


def _model(sizes, act, dtype, ffg, eta, seed):
    from predicitivecoding_amd import GenerativeSnapshot, PcDeviceModel
    W, b, P = make_net(sizes, seed=seed, bias_scale=0.1)
    snap = GenerativeSnapshot(sizes, act, eta, 0.0, bool(ffg), W, b, list(P))
    return PcDeviceModel(snap, dtype)


def _run(name, model, x, steps):
    """One call of `name` through the C ABI on library device buffers (the
    outputs start as NaN, so a value the call does not write shows)."""
    from predicitivecoding_amd import DeviceTensor
    from predicitivecoding_amd._native import call
    B = x.shape[0]
    nan = np.float32("nan")
    bufs = [DeviceTensor.from_host(x),
            DeviceTensor.from_host(np.full((B, model.sizes[-1]), nan, np.float32)),
            DeviceTensor.from_host(np.full((B * sum(model.sizes),), nan, np.float32)),
            DeviceTensor.from_host(np.full((steps, B), nan, np.float32))]
    try:
        dx, top, states, energy = bufs
        call(name, model.handle, dx.ptr, B, steps, top.ptr, states.ptr, energy.ptr, None)
        call("pcd_device_synchronize")
        return top.to_host(), states.to_host(), energy.to_host()
    finally:
        for t in bufs:
            t.free()


@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_matches_relax_bit_for_bit(case):
    sizes, act, dtype, ffg, eta, batches = CASES[case]
    print(f"noalloc case {case}: {sizes} act {act} {dtype} ffg {ffg} batches {batches}", flush=True)
    # another model's call first: it leaves its states in the shared scratch
    other = _model([300, 700, 50], 4, "bf16", 0, 0.05, seed=99)
    try:
        _run("pcd_pc_relax_noalloc", other, make_inputs(200, 300, seed=98), 3)
    finally:
        other.close()
    model = _model(sizes, act, dtype, ffg, eta, seed=case)
    try:
        for k, B in enumerate(batches):
            x = make_inputs(B, sizes[0], seed=10 * case + k)
            steps = 12 - 5 * k
            want = _run("pcd_pc_relax", model, x, steps)
            got = _run("pcd_pc_relax_noalloc", model, x, steps)
            for what, g, w in zip(("top", "states", "energy"), got, want):
                assert np.isfinite(w).all(), what
                assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), \
                    (what, B, float(np.max(np.abs(g - w))))
            print(f"  B={B} T={steps}: top, states and energies bit-identical", flush=True)
    finally:
        model.close()


def test_noalloc_refuses_a_batch_beyond_its_scratch():
    from predicitivecoding_amd import DeviceTensor
    from predicitivecoding_amd._native import last_error, lib
    sizes = [784, 256, 256, 10]
    model = _model(sizes, 1, "f32", 0, 0.1, seed=0)
    B = 20000   # its states alone need ~115 MB, beyond the 64 MiB array
    dx = DeviceTensor.from_host(np.zeros((B, sizes[0]), np.float32))
    top = DeviceTensor.from_host(np.zeros((B, sizes[-1]), np.float32))
    try:
        st = lib().pcd_pc_relax_noalloc(model.handle, dx.ptr, B, 5, top.ptr, None, None, None)
        assert st == 4, st
        assert "scratch" in last_error() and "use pcd_pc_relax" in last_error()
        assert float(np.abs(top.to_host()).max()) == 0.0   # nothing was launched
    finally:
        dx.free()
        top.free()
        model.close()


def test_noalloc_calls_on_two_streams_are_ordered():
    # Two models' calls queued back to back on two streams, with no
    # synchronisation between them, share the device's one scratch array: the
    # library orders them (the second stream waits on the first call's event),
    # so each result still equals pcd_pc_relax's bit for bit.
    from predicitivecoding_amd import DeviceTensor, Stream
    from predicitivecoding_amd._native import call
    specs = [([1024, 2048, 1024, 64], 4, "bf16", 512, 9), ([784, 256, 256, 10], 1, "f32", 64, 7)]
    models = [_model(sizes, act, dtype, 0, 0.05, seed=70 + i) for i, (sizes, act, dtype, _, _) in enumerate(specs)]
    streams = [Stream(), Stream()]
    bufs = []
    try:
        wants, outs = [], []
        for (sizes, _, _, B, steps), model in zip(specs, models):
            x = make_inputs(B, sizes[0], seed=B)
            wants.append(_run("pcd_pc_relax", model, x, steps))
            dx = DeviceTensor.from_host(x)
            top = DeviceTensor.from_host(np.full((B, sizes[-1]), np.float32("nan"), np.float32))
            states = DeviceTensor.from_host(np.full((B * sum(sizes),), np.float32("nan"), np.float32))
            energy = DeviceTensor.from_host(np.full((steps, B), np.float32("nan"), np.float32))
            bufs += [dx, top, states, energy]
            outs.append((dx, top, states, energy))
        for rep in range(3):
            for (sizes, _, _, B, steps), model, stream, (dx, top, states, energy) in zip(specs, models, streams, outs):
                call("pcd_pc_relax_noalloc", model.handle, dx.ptr, B, steps, top.ptr, states.ptr, energy.ptr,
                     stream.handle)
            for stream in streams:
                stream.synchronize()
            for i, (want, (_, top, states, energy)) in enumerate(zip(wants, outs)):
                for what, g, w in zip(("top", "states", "energy"), (top.to_host(), states.to_host(),
                                                                    energy.to_host()), want):
                    assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (rep, i, what)
            print(f"two streams, round {rep}: both calls bit-identical to pcd_pc_relax", flush=True)
    finally:
        for t in bufs:
            t.free()
        for stream in streams:
            stream.close()
        for model in models:
            model.close()
