"""The reference-API drop-in, BatchedPcForward.infer_get_top_batch, on the GPU.

Mirrors PredicitiveCoding.UnitTests/BatchedPcForwardTests.cs: the [6,10,4]
tanh network (eta 0.1, eta_w 0.05) trained on two patterns, inputs uniform in
[-1, 1], and the reference's bounds |a-b| <= tol*(1+|b|):
  batched == per-sample InferGetTop          1e-3   (:44-72, :74-92 with FFG)
  mixed tracks float                          5e-2   (:94-111)
and, tighter, this build's own bars: fp32 against the fp32 oracle 1e-4, and
16-bit operands against the oracle with the same operand rounding 2e-3.
"""
import gc

import numpy as np
import pytest

from tests.netgen import close, make_inputs, make_net, max_rel

pytestmark = pytest.mark.gpu

SIZES = [6, 10, 4]


def _trained_snapshot(oracle, seed, ffg=False):
    """The reference test's network: Xavier-normal weights, then 30 rounds of
    Learn(x0 = 0 -> class 0) and Learn(x1 = 1 -> class 1) with 10 steps
    (BatchedPcForwardTests.cs:47-56), here with the oracle's learning step."""
    from predicitivecoding_amd import GenerativeSnapshot
    W, b, P = make_net(SIZES, seed=seed)
    x0, x1 = np.zeros((1, 6), np.float32), np.ones((1, 6), np.float32)
    y0, y1 = np.eye(4, dtype=np.float32)[:1], np.eye(4, dtype=np.float32)[1:2]
    for _ in range(30):
        for x, y in ((x0, y0), (x1, y1)):
            W, b, _ = oracle.learn(SIZES, "tanh", 0.1, W, b, P, x, y, 10, 0.05)
    W = [np.ascontiguousarray(w, np.float32) for w in W]
    b = [np.ascontiguousarray(v, np.float32) for v in b]
    return GenerativeSnapshot(SIZES, 1, 0.1, 0.0, ffg, W, b, list(P)), W, b, P


def _inputs(count, seed):
    return [row for row in make_inputs(count, 6, seed=seed, dist="uniform11")]


def test_batch_matches_per_sample_infer_get_top(oracle):
    from predicitivecoding_amd import BatchedPcForward
    snap, W, b, P = _trained_snapshot(oracle, seed=0)
    inputs = _inputs(5, seed=3)
    batched = BatchedPcForward.infer_get_top_batch(snap, inputs, 15)
    assert len(batched) == 5 and all(t.shape == (4,) and t.dtype == np.float32 for t in batched)
    got = np.stack(batched)
    x = np.stack(inputs)
    per_sample, _, _ = oracle.persample_relax_f64(SIZES, "tanh", 0.1, W, b, P, x, 15)
    ref32, _, _ = oracle.batched_relax(SIZES, "tanh", 0.1, W, b, P, x, 15)
    print(f"drop-in fp32: vs per-sample f64 {max_rel(got, per_sample):.2e}, vs oracle {max_rel(got, ref32):.2e}",
          flush=True)
    assert close(got, per_sample, 1e-3)
    assert max_rel(got, ref32) < 1e-4


def test_batch_with_feedforward_gist_matches_per_sample(oracle):
    from predicitivecoding_amd import BatchedPcForward, GenerativeSnapshot
    W, b, P = make_net(SIZES, seed=1)
    snap = GenerativeSnapshot(SIZES, 1, 0.1, 0.0, True, W, b, list(P))
    inputs = _inputs(4, seed=5)
    got = np.stack(BatchedPcForward.infer_get_top_batch(snap, inputs, 10))
    x = np.stack(inputs)
    per_sample, _, _ = oracle.persample_relax_f64(SIZES, "tanh", 0.1, W, b, P, x, 10, ffg=True)
    ref32, _, _ = oracle.batched_relax(SIZES, "tanh", 0.1, W, b, P, x, 10, ffg=True)
    assert close(got, per_sample, 1e-3)
    assert max_rel(got, ref32) < 1e-4


@pytest.mark.parametrize("dtype", [None, "bf16"])
def test_mixed_batch_tracks_float_batch(oracle, dtype):
    # mixed=True is fp16 operands (Gemm.cs:44-60); dtype="bf16" selects bf16
    from predicitivecoding_amd import BatchedPcForward
    snap, W, b, P = _trained_snapshot(oracle, seed=2)
    inputs = _inputs(4, seed=7)
    full = np.stack(BatchedPcForward.infer_get_top_batch(snap, inputs, 15))
    mixed = np.stack(BatchedPcForward.infer_get_top_batch(snap, inputs, 15, mixed=True, dtype=dtype))
    x = np.stack(inputs)
    same, _, _ = oracle.batched_relax(SIZES, "tanh", 0.1, W, b, P, x, 15, round_mode=dtype or "f16")
    print(f"drop-in mixed/{dtype or 'f16'}: vs float {max_rel(mixed, full):.2e}, "
          f"vs same rounding {max_rel(mixed, same):.2e}", flush=True)
    assert close(mixed, full, 5e-2)
    assert max_rel(mixed, same) < 2e-3
    assert not np.array_equal(mixed, full)   # the 16-bit path really ran


def test_drop_in_releases_device_models_with_their_snapshots(oracle):
    # The drop-in keeps one device model per live snapshot and operand type;
    # a snapshot that is collected takes its model (W, W^T, workspaces,
    # graphs) with it, so a caller exporting snapshot after snapshot does not
    # accumulate device memory.
    from predicitivecoding_amd import BatchedPcForward, GenerativeSnapshot
    gc.collect()
    base = BatchedPcForward.cached_models()
    inputs = _inputs(3, seed=9)
    keep = None
    for k in range(6):
        W, b, P = make_net(SIZES, seed=40 + k)
        snap = GenerativeSnapshot(SIZES, 1, 0.1, 0.0, False, W, b, list(P))
        top = np.stack(BatchedPcForward.infer_get_top_batch(snap, inputs, 5))
        ref, _, _ = oracle.batched_relax(SIZES, "tanh", 0.1, W, b, P, np.stack(inputs), 5)
        assert max_rel(top, ref) < 1e-4
        if k == 0:
            keep = snap
            BatchedPcForward.infer_get_top_batch(snap, inputs, 5, mixed=True)
        del snap
        gc.collect()
        assert BatchedPcForward.cached_models() == base + 2   # keep's f32 and f16 models only
    # the kept snapshot's models are still the cached ones and still work
    again = np.stack(BatchedPcForward.infer_get_top_batch(keep, inputs, 5))
    assert BatchedPcForward.cached_models() == base + 2
    W, b, P = make_net(SIZES, seed=40)
    ref, _, _ = oracle.batched_relax(SIZES, "tanh", 0.1, W, b, P, np.stack(inputs), 5)
    assert max_rel(again, ref) < 1e-4
    del keep
    gc.collect()
    assert BatchedPcForward.cached_models() == base


def test_drop_in_sees_the_snapshot_as_made(oracle):
    # An in-place edit of the arrays a snapshot was made from, after its first
    # call, must not leave the cached device model silently out of step with
    # the snapshot: the snapshot holds its own read-only copies, so its
    # weights (and the device model's) are the ones it was made with, and a
    # new snapshot of the edited arrays settles with the edit.
    from predicitivecoding_amd import BatchedPcForward, GenerativeSnapshot
    W, b, P = make_net(SIZES, seed=61)
    inputs = _inputs(4, seed=62)
    x = np.stack(inputs)
    snap = GenerativeSnapshot(SIZES, 1, 0.1, 0.0, False, W, b, list(P))
    first = np.stack(BatchedPcForward.infer_get_top_batch(snap, inputs, 8))
    W[0][:] *= 3.0                   # the caller edits its own arrays in place
    with pytest.raises(ValueError):
        snap.weights[0][0, 0] = 1.0  # and cannot edit the snapshot's
    again = np.stack(BatchedPcForward.infer_get_top_batch(snap, inputs, 8))
    assert np.array_equal(first, again)
    ref, _, _ = oracle.batched_relax(SIZES, "tanh", 0.1, [w for w in snap.weights], list(snap.biases), P, x, 8)
    assert max_rel(again, ref) < 1e-4
    edited = GenerativeSnapshot(SIZES, 1, 0.1, 0.0, False, W, b, list(P))
    new = np.stack(BatchedPcForward.infer_get_top_batch(edited, inputs, 8))
    ref2, _, _ = oracle.batched_relax(SIZES, "tanh", 0.1, W, b, P, x, 8)
    assert max_rel(new, ref2) < 1e-4
    assert not np.allclose(new, first)


def _allocating_top(model, x, steps):
    """The top through per-call device buffers and synchronous copies."""
    from predicitivecoding_amd import DeviceTensor
    from predicitivecoding_amd.device import DeviceRuntime
    dx = DeviceTensor.from_host(x)
    top = DeviceTensor((x.shape[0], model.sizes[-1]))
    try:
        model.relax_device(dx.ptr, x.shape[0], steps, top.ptr)
        DeviceRuntime.synchronize()
        return top.to_host()
    finally:
        dx.free()
        top.free()


def test_staged_top_path_matches_allocating_path(oracle):
    # Top-only host settlings go through the model's pinned staging buffers,
    # grown to the largest batch seen.  Batches that grow and shrink give the
    # same bits as per-call device buffers, and the oracle's values.
    from predicitivecoding_amd import BatchedPcForward, PcDeviceModel
    snap, W, b, P = _trained_snapshot(oracle, seed=41)
    m = PcDeviceModel(snap, "f32")
    try:
        for B in (5, 33, 12, 70, 1, 70):
            x = make_inputs(B, 6, seed=100 + B, dist="uniform11")
            staged, _, _ = m.relax(x, 8)
            assert np.array_equal(staged, _allocating_top(m, x, 8)), B
            ref, _, _ = oracle.batched_relax(SIZES, "tanh", 0.1, W, b, P, x, 8)
            assert max_rel(staged, ref) < 1e-4, B
            rows = BatchedPcForward.infer_get_top_batch(snap, list(x), 8)
            assert len(rows) == B and all(np.array_equal(r, staged[i]) for i, r in enumerate(rows))
    finally:
        m.close()


def test_staged_top_path_under_concurrent_callers(oracle):
    # Two threads settle on one model at once: one holds the staging set, the
    # other takes the allocating path; both get the single-caller bits.
    import threading

    from predicitivecoding_amd import PcDeviceModel, Stream
    snap, _, _, _ = _trained_snapshot(oracle, seed=42)
    m = PcDeviceModel(snap, "f32")
    xs = [make_inputs(40, 6, seed=200 + t, dist="uniform11") for t in range(2)]
    want = [m.relax(x, 9)[0] for x in xs]
    got, errors = [[None] * 6 for _ in range(2)], []

    def worker(t):
        s = Stream()
        try:
            for i in range(6):
                got[t][i] = m.relax(xs[t], 9, stream=s)[0]
        except Exception as e:   # reported below
            errors.append(e)
        finally:
            s.close()

    try:
        threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
        for th in threads:
            th.start()
        for th in threads:
            th.join(timeout=60)
        assert not errors, errors
        for t in range(2):
            assert all(np.array_equal(g, want[t]) for g in got[t])
    finally:
        m.close()


def test_graph_recording_beside_synchronous_copies_on_another_thread(oracle):
    # HIP refuses a legacy-stream copy (pcd_memcpy) while any stream of the
    # process records a graph, and then invalidates the recording; the library
    # keeps its recordings and its synchronous copies apart.  One thread
    # records a new graph per call (a new step count each time) while another
    # copies to and from the device the whole time; both get their bits.
    import threading

    from predicitivecoding_amd import PcDeviceModel, Stream
    from predicitivecoding_amd.device import DeviceTensor
    snap, _, _, _ = _trained_snapshot(oracle, seed=43)
    m = PcDeviceModel(snap, "f32")
    x = make_inputs(40, 6, seed=300, dist="uniform11")
    steps = list(range(3, 15))
    want = [m.relax(x, t)[0] for t in steps]
    errors, stop = [], threading.Event()

    def copier():
        buf = np.arange(4096, dtype=np.float32)
        try:
            while not stop.is_set():
                t = DeviceTensor.from_host(buf)
                try:
                    if not np.array_equal(t.to_host(), buf):
                        raise AssertionError("copy came back changed")
                finally:
                    t.free()
        except Exception as e:   # reported below
            errors.append(e)

    th = threading.Thread(target=copier)
    th.start()
    s = Stream()
    got = []
    try:
        for t in steps:
            got.append(m.relax(x, t, stream=s)[0])
    except Exception as e:   # reported below
        errors.append(e)
    finally:
        stop.set()
        th.join(timeout=60)
        s.close()
        m.close()
    assert not errors, errors
    assert all(np.array_equal(g, w) for g, w in zip(got, want))
