"""BatchedPcForward on MI355X: the reference entry point over libpcdevice_hip.

``BatchedPcForward.infer_get_top_batch`` keeps the signature, argument checks
and semantics of BatchedPcForward.InferGetTopBatch
(PredictiveCoding.Device/BatchedPcForward.cs:36-139): settle every input from
zero free states with layer 0 clamped, return the top latent per sample.
``mixed=True`` selects 16-bit GEMM operands with fp32 accumulation; like the
reference (Gemm.cs:44-60) that is fp16 unless ``dtype="bf16"`` is asked for.

``PcDeviceModel`` is the device-resident model (pcd_pc_model_create) with the
extended entry points: all final states, per-step energies, device-pointer
I/O for benchmarks, and ragged request batches with early exit.
"""
from __future__ import annotations

import ctypes
import threading
import weakref

import numpy as np

from . import _native
from ._native import DTYPE, EXIT, MEMCPY, call
from .device import DeviceTensor, Stream
from .effort import EffortLevel, EffortPresets
from .errors import ArgumentException, ArgumentNullException, ArgumentOutOfRangeException
from .snapshot import GenerativeSnapshot


def _check_ragged_tables(offs: np.ndarray, steps: np.ndarray) -> None:
    """Host tables of a ragged call: R >= 1 requests, R + 1 strictly increasing
    row offsets from 0 (the library reads row_offsets[R]), budgets >= 1."""
    R = len(steps)
    if R < 1:
        raise ArgumentException("Empty batch.")
    if len(offs) != R + 1 or offs[0] != 0 or np.any(np.diff(offs) < 1):
        raise ArgumentException("row_offsets must start at 0, increase strictly and end at the row count")
    if np.any(steps < 1):
        raise ArgumentOutOfRangeException("steps")


def _free_stage(ptrs: list) -> None:
    """Returns a staging set's buffers to the library's pools (pinned host
    pair first, then the device pair)."""
    if ptrs:
        h_in, h_out, d_in, d_out = ptrs
        _native.lib().pcd_host_free(ctypes.c_void_p(h_in))
        _native.lib().pcd_host_free(ctypes.c_void_p(h_out))
        _native.lib().pcd_free_async(ctypes.c_void_p(d_in), None)
        _native.lib().pcd_free_async(ctypes.c_void_p(d_out), None)
        ptrs.clear()


class _TopStage:
    """Pinned host and device buffers a model keeps for its top-only host
    settlings (the drop-in's calls): the input rows are written straight into
    pinned memory, and the input copy, the settling and the top copy queue on
    one stream behind one synchronisation, with nothing allocated per call.
    Grown to the largest batch seen; one caller at a time (`lock`)."""

    def __init__(self, s0: int, s_top: int):
        self.s0, self.s_top = s0, s_top
        self.rows = 0
        self.ptrs: list = []
        self.lock = threading.Lock()
        self._finalizer = weakref.finalize(self, _free_stage, self.ptrs)

    def ensure(self, rows: int) -> None:
        if rows <= self.rows:
            return
        cap = max(rows, 2 * self.rows)
        _free_stage(self.ptrs)
        self.rows = 0
        got = []
        try:
            for nbytes, fn in ((cap * self.s0 * 4, "pcd_host_alloc"), (cap * self.s_top * 4, "pcd_host_alloc")):
                p = ctypes.c_void_p()
                call(fn, ctypes.byref(p), nbytes)
                got.append(p.value)
            for nbytes in (cap * self.s0 * 4, cap * self.s_top * 4):
                p = ctypes.c_void_p()
                call("pcd_malloc_async", ctypes.byref(p), nbytes, None)
                got.append(p.value)
            call("pcd_device_synchronize")   # the pool's blocks are ready for any stream
        except BaseException:
            for i, q in enumerate(got):
                if i < 2:
                    _native.lib().pcd_host_free(ctypes.c_void_p(q))
                else:
                    _native.lib().pcd_free_async(ctypes.c_void_p(q), None)
            raise
        self.ptrs.extend(got)
        self.rows = cap

    def view(self, which: int, rows: int, cols: int) -> np.ndarray:
        """[rows x cols] float32 array over pinned buffer `which` (0 input, 1 top)."""
        buf = (ctypes.c_float * (rows * cols)).from_address(self.ptrs[which])
        return np.frombuffer(buf, dtype=np.float32).reshape(rows, cols)

    def close(self) -> None:
        with self.lock:
            self._finalizer()
            self.rows = 0


class PcDeviceModel:
    """A GenerativeSnapshot uploaded to the current GPU in one operand dtype."""

    def __init__(self, snapshot: GenerativeSnapshot, dtype: str = "f32"):
        if dtype not in DTYPE:
            raise ArgumentException(f"dtype must be one of {sorted(DTYPE)}")
        # the weights are copied to the device: no reference to the snapshot
        # is kept (the drop-in's cache frees a model when its snapshot dies)
        self.dtype = dtype
        L = len(snapshot.layer_sizes)
        self.sizes = list(snapshot.layer_sizes)
        sizes = (ctypes.c_int * L)(*self.sizes)
        wp = (ctypes.c_void_p * (L - 1))(*[w.ctypes.data for w in snapshot.weights])
        bp = (ctypes.c_void_p * (L - 1))(*[b.ctypes.data for b in snapshot.biases])
        prec = (ctypes.c_float * L)(*snapshot.precisions)
        h = ctypes.c_void_p()
        call("pcd_pc_model_create", sizes, L, int(snapshot.activation), float(snapshot.state_learning_rate),
             float(snapshot.activity_regularization), int(bool(snapshot.use_feedforward_gist_init)),
             wp, bp, prec, DTYPE[dtype], ctypes.byref(h))
        self.handle = h.value
        self._finalizer = weakref.finalize(self, _native.lib().pcd_pc_model_destroy, self.handle)
        self._stage = _TopStage(self.sizes[0], self.sizes[-1])

    def close(self) -> None:
        self._stage.close()
        self._finalizer()
        self.handle = None

    def set_option(self, name: str, value: int) -> None:
        call("pcd_pc_set_option", self.handle, name.encode(), int(value))

    def profile_result(self):
        e, u, n = ctypes.c_float(), ctypes.c_float(), ctypes.c_int()
        call("pcd_pc_profile_result", self.handle, ctypes.byref(e), ctypes.byref(u), ctypes.byref(n))
        return e.value, u.value, n.value

    # ---------------------------------------------------------- device I/O

    def relax_device(self, x0_ptr: int, batch: int, steps: int, out_top_ptr: int,
                     out_states_ptr: int | None = None, out_energy_ptr: int | None = None,
                     stream: Stream | None = None) -> None:
        """pcd_pc_relax on device pointers, queued on `stream` (no sync)."""
        call("pcd_pc_relax", self.handle, x0_ptr, int(batch), int(steps), out_top_ptr,
             out_states_ptr, out_energy_ptr, stream.handle if stream else None)

    # ------------------------------------------------------------ host I/O

    def relax(self, x0: np.ndarray, steps: int, want_states: bool = False, want_energy: bool = False,
              stream: Stream | None = None):
        """Settle a [batch x s_0] host batch; returns (top, states, energy)."""
        x0 = np.ascontiguousarray(x0, dtype=np.float32)
        if x0.ndim != 2 or x0.shape[1] != self.sizes[0]:
            raise ArgumentException(f"inputs must be [batch x {self.sizes[0]}]")
        B = x0.shape[0]
        if B < 1:
            raise ArgumentException("Empty batch.")
        if steps < 1:
            raise ArgumentOutOfRangeException("inferenceSteps")
        if not want_states and not want_energy:
            top = self._relax_top_staged(B, steps, lambda v: np.copyto(v, x0), stream)
            if top is not None:
                return top, None, None
        dx = DeviceTensor.from_host(x0)
        top = DeviceTensor((B, self.sizes[-1]))
        st = DeviceTensor((B * sum(self.sizes),)) if want_states else None
        en = DeviceTensor((steps, B)) if want_energy else None
        try:
            self.relax_device(dx.ptr, B, steps, top.ptr, st.ptr if st else None, en.ptr if en else None, stream)
            if stream:
                stream.synchronize()
            else:
                call("pcd_device_synchronize")
            top_h = top.to_host()
            states = None
            if st is not None:
                flat, states, off = st.to_host(), [], 0
                for s in self.sizes:
                    states.append(flat[off:off + B * s].reshape(B, s))
                    off += B * s
            energy = en.to_host() if en is not None else None
        finally:
            for t in (dx, top, st, en):
                if t is not None:
                    t.free()
        return top_h, states, energy

    def _relax_top_staged(self, B: int, steps: int, fill, stream: Stream | None = None):
        """Top-only settling through the model's staging buffers: `fill` writes
        the [B x s_0] input rows into pinned memory; returns the [B x s_top]
        top as a new array, or None when another caller holds the staging set
        (that caller's call then takes the allocating path)."""
        st = self._stage
        if not st.lock.acquire(blocking=False):
            return None
        try:
            st.ensure(B)
            h_in, h_out, d_in, d_out = st.ptrs
            fill(st.view(0, B, self.sizes[0]))
            sh = stream.handle if stream else None
            call("pcd_memcpy_async", d_in, h_in, B * self.sizes[0] * 4, MEMCPY["h2d"], sh)
            self.relax_device(d_in, B, steps, d_out, stream=stream)
            call("pcd_memcpy_async", h_out, d_out, B * self.sizes[-1] * 4, MEMCPY["d2h"], sh)
            call("pcd_stream_synchronize", sh)
            return st.view(1, B, self.sizes[-1]).copy()
        finally:
            st.lock.release()

    def relax_ragged_device(self, x0_ptr: int, row_offsets, steps, top_ptr: int, exit_rule: str = "none",
                            exit_threshold: float = 0.0, stream: Stream | None = None):
        """pcd_pc_relax_ragged on device input/output pointers (the call
        synchronises its stream); returns (steps_used, final_energy)."""
        offs = np.ascontiguousarray(row_offsets, dtype=np.int32)
        st = np.ascontiguousarray(steps, dtype=np.int32)
        R = len(st)
        _check_ragged_tables(offs, st)
        used = np.zeros(R, dtype=np.int32)
        fe = np.zeros(R, dtype=np.float32)
        if exit_rule not in EXIT:
            raise ArgumentException(f"exit_rule must be one of {sorted(EXIT)}")
        call("pcd_pc_relax_ragged", self.handle, x0_ptr,
             offs.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), st.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
             R, EXIT[exit_rule], float(exit_threshold), used.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
             top_ptr, fe.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), stream.handle if stream else None)
        return used, fe

    def relax_ragged(self, x0_packed: np.ndarray, row_offsets, steps, exit_rule: str = "none",
                     exit_threshold: float = 0.0, stream: Stream | None = None):
        """Ragged requests with early exit; returns (steps_used, final_energy, top)."""
        x0 = np.ascontiguousarray(x0_packed, dtype=np.float32)
        offs = np.ascontiguousarray(row_offsets, dtype=np.int32)
        st = np.ascontiguousarray(steps, dtype=np.int32)
        R = len(st)
        _check_ragged_tables(offs, st)
        if offs[-1] != x0.shape[0]:
            raise ArgumentException("row_offsets must start at 0, increase strictly and end at the row count")
        if exit_rule not in EXIT:
            raise ArgumentException(f"exit_rule must be one of {sorted(EXIT)}")
        rows = int(offs[-1])
        dx = DeviceTensor.from_host(x0)
        top = DeviceTensor((rows, self.sizes[-1]))
        used = np.zeros(R, dtype=np.int32)
        fe = np.zeros(R, dtype=np.float32)
        try:
            call("pcd_pc_relax_ragged", self.handle, dx.ptr,
                 offs.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), st.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                 R, EXIT[exit_rule], float(exit_threshold), used.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                 top.ptr, fe.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), stream.handle if stream else None)
            top_h = top.to_host()
        finally:
            dx.free()
            top.free()
        return used, fe, top_h


    # ------------------------------------- clamped settling, classes, learning

    def _batch_in(self, x, cols, name):
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != cols:
            raise ArgumentException(f"{name} must be [batch x {cols}]")
        if x.shape[0] < 1:
            raise ArgumentException("Empty batch.")
        return x

    def _sync(self, stream):
        if stream:
            stream.synchronize()
        else:
            call("pcd_device_synchronize")

    def relax_clamped(self, x0: np.ndarray, top: np.ndarray, steps: int, want_states: bool = False,
                      stream: Stream | None = None):
        """pcd_pc_relax_clamped on host arrays: input and top clamped (Network.InferCore
        with a label).  Returns (states list or None, energy [steps x batch])."""
        x0 = self._batch_in(x0, self.sizes[0], "inputs")
        B = x0.shape[0]
        top = np.ascontiguousarray(top, dtype=np.float32).reshape(B, self.sizes[-1])
        if steps < 1:
            raise ArgumentOutOfRangeException("inferenceSteps")
        dx, dt = DeviceTensor.from_host(x0), DeviceTensor.from_host(top)
        st = DeviceTensor((B * sum(self.sizes),)) if want_states else None
        en = DeviceTensor((steps, B))
        try:
            call("pcd_pc_relax_clamped", self.handle, dx.ptr, dt.ptr, B, int(steps), st.ptr if st else None, en.ptr,
                 stream.handle if stream else None)
            self._sync(stream)
            states = None
            if st is not None:
                flat, states, off = st.to_host(), [], 0
                for s in self.sizes:
                    states.append(flat[off:off + B * s].reshape(B, s))
                    off += B * s
            energy = en.to_host()
        finally:
            for t in (dx, dt, st, en):
                if t is not None:
                    t.free()
        return states, energy

    def classify_device(self, x0_ptr: int, batch: int, steps: int, class_energies_ptr: int | None = None,
                        class_ptr: int | None = None, energy_ptr: int | None = None,
                        stream: Stream | None = None) -> None:
        """pcd_pc_classify on device pointers, queued on `stream` (no sync)."""
        call("pcd_pc_classify", self.handle, x0_ptr, int(batch), int(steps), class_energies_ptr, class_ptr,
             energy_ptr, stream.handle if stream else None)

    def classify(self, x0: np.ndarray, steps: int, stream: Stream | None = None):
        """Minimum-energy classification of a host batch (Network.ClassEnergies and
        PredictWithEnergy per sample).  Returns (class_energies [B x C], class [B],
        energy [B])."""
        x0 = self._batch_in(x0, self.sizes[0], "inputs")
        if steps < 1:
            raise ArgumentOutOfRangeException("inferenceSteps")
        B, C = x0.shape[0], self.sizes[-1]
        dx = DeviceTensor.from_host(x0)
        ce = DeviceTensor((B, C))
        cls = DeviceTensor((B,), dtype=np.int32)
        be = DeviceTensor((B,))
        try:
            self.classify_device(dx.ptr, B, steps, ce.ptr, cls.ptr, be.ptr, stream)
            self._sync(stream)
            out = ce.to_host(), cls.to_host(), be.to_host()
        finally:
            for t in (dx, ce, cls, be):
                t.free()
        return out

    def classify_adaptive_device(self, x0_ptr: int, batch: int, max_steps: int, epsilon: float,
                                 class_energies_ptr: int | None = None, class_steps_ptr: int | None = None,
                                 class_ptr: int | None = None, energy_ptr: int | None = None,
                                 steps_used_ptr: int | None = None, stream: Stream | None = None) -> None:
        """pcd_pc_classify_adaptive on device pointers, queued on `stream` (no sync)."""
        call("pcd_pc_classify_adaptive", self.handle, x0_ptr, int(batch), int(max_steps), float(epsilon),
             class_energies_ptr, class_steps_ptr, class_ptr, energy_ptr, steps_used_ptr,
             stream.handle if stream else None)

    def classify_adaptive(self, x0: np.ndarray, max_steps: int, epsilon: float, stream: Stream | None = None):
        """Network.PredictAdaptive (Network.cs:803-840) for every sample of a host
        batch.  Returns (class_energies [B x C], class_steps [B x C], class [B],
        energy [B], steps_used [B])."""
        x0 = self._batch_in(x0, self.sizes[0], "inputs")
        if max_steps < 1:
            raise ArgumentOutOfRangeException("maxSteps")
        B, C = x0.shape[0], self.sizes[-1]
        dx = DeviceTensor.from_host(x0)
        outs = [DeviceTensor((B, C)), DeviceTensor((B, C), dtype=np.int32), DeviceTensor((B,), dtype=np.int32),
                DeviceTensor((B,)), DeviceTensor((B,), dtype=np.int32)]
        try:
            self.classify_adaptive_device(dx.ptr, B, max_steps, epsilon, *[t.ptr for t in outs], stream=stream)
            self._sync(stream)
            res = tuple(t.to_host() for t in outs)
        finally:
            for t in [dx, *outs]:
                t.free()
        return res

    def predict_adaptive(self, x0: np.ndarray, effort: EffortLevel, stream: Stream | None = None):
        """PredictAdaptive with a named effort preset (Network.cs:843-847):
        returns (class [B], energy [B], steps_used [B])."""
        max_steps, epsilon = EffortPresets.for_level(effort)
        _, _, cls, energy, used = self.classify_adaptive(x0, max_steps, epsilon, stream)
        return cls, energy, used

    def learn_device(self, x0_ptr: int, labels_ptr: int, batch: int, steps: int, eta_w: float,
                     weight_decay: float = 0.0, energy_ptr: int | None = None, stream: Stream | None = None) -> None:
        """pcd_pc_learn on device pointers, queued on `stream` (no sync)."""
        call("pcd_pc_learn", self.handle, x0_ptr, labels_ptr, int(batch), int(steps), float(eta_w),
             float(weight_decay), energy_ptr, stream.handle if stream else None)

    def learn(self, x0: np.ndarray, labels: np.ndarray, steps: int, eta_w: float, weight_decay: float = 0.0,
              stream: Stream | None = None, hidden=None, want_hidden: bool = False):
        """Network.Learn on a host batch (the sum of the per-sample updates);
        returns each sample's energy at the last step.  `hidden` (a list of
        [B x s_l] arrays for l = 1..L-2, or None for zeros) is the hidden state
        the settling starts from, as the reference's network holds it between
        calls (pcd_pc_learn_warm); with want_hidden the settled hidden states
        come back too, as (energy, hidden)."""
        x0 = self._batch_in(x0, self.sizes[0], "inputs")
        B = x0.shape[0]
        labels = np.ascontiguousarray(labels, dtype=np.float32).reshape(B, self.sizes[-1])
        if steps < 1:
            raise ArgumentOutOfRangeException("inferenceSteps")
        hs = self.sizes[1:-1]
        if hidden is not None:
            hidden = list(hidden)
            if len(hidden) != len(hs):
                raise ArgumentException(f"hidden must hold {len(hs)} layers")
            hidden = [np.ascontiguousarray(h, dtype=np.float32).reshape(B, s) for h, s in zip(hidden, hs)]
        dx, dl = DeviceTensor.from_host(x0), DeviceTensor.from_host(labels)
        en = DeviceTensor((B,))
        nh = B * sum(hs)
        dh_in = DeviceTensor.from_host(np.concatenate([h.ravel() for h in hidden])) if hidden and nh else None
        dh_out = DeviceTensor((nh,)) if want_hidden and nh else None
        try:
            if dh_in is None and dh_out is None:
                self.learn_device(dx.ptr, dl.ptr, B, steps, eta_w, weight_decay, en.ptr, stream)
            else:
                call("pcd_pc_learn_warm", self.handle, dx.ptr, dl.ptr, dh_in.ptr if dh_in else None,
                     dh_out.ptr if dh_out else None, B, int(steps), float(eta_w), float(weight_decay), en.ptr,
                     stream.handle if stream else None)
            self._sync(stream)
            energy = en.to_host()
            out = []
            if want_hidden:
                flat, off = dh_out.to_host() if dh_out else np.zeros(0, np.float32), 0
                for s in hs:
                    out.append(flat[off:off + B * s].reshape(B, s))
                    off += B * s
        finally:
            for t in (dx, dl, en, dh_in, dh_out):
                if t is not None:
                    t.free()
        return (energy, out) if want_hidden else energy

    def load_record(self, layer: int, record: bytes) -> None:
        """pcd_pc_model_load_record: one LayerSerializer record (the layer's
        persisted bytes) into the device operands."""
        buf = ctypes.create_string_buffer(bytes(record), len(record))
        call("pcd_pc_model_load_record", self.handle, int(layer), buf, len(record))

    @classmethod
    def from_records(cls, records, activation: int, eta: float, act_reg: float = 0.0, ffg: bool = False,
                     dtype: str = "f32") -> "PcDeviceModel":
        """A device model straight from the layers' records (layer 0 first), as
        Network reopens its store: sizes and precisions from the record headers,
        weights uploaded in their stored format."""
        import struct
        sizes = [struct.unpack_from("<i", r, 0)[0] for r in records]
        precisions = [struct.unpack_from("<f", r, 8)[0] for r in records]
        self = cls.__new__(cls)
        self.dtype = dtype
        self.sizes = sizes
        L = len(sizes)
        if dtype not in DTYPE:
            raise ArgumentException(f"dtype must be one of {sorted(DTYPE)}")
        h = ctypes.c_void_p()
        call("pcd_pc_model_create", (ctypes.c_int * L)(*sizes), L, int(activation), float(eta), float(act_reg),
             int(bool(ffg)), None, None, (ctypes.c_float * L)(*precisions), DTYPE[dtype], ctypes.byref(h))
        self.handle = h.value
        self._finalizer = weakref.finalize(self, _native.lib().pcd_pc_model_destroy, self.handle)
        self._stage = _TopStage(self.sizes[0], self.sizes[-1])
        for l, r in enumerate(records):
            self.load_record(l, r)
        return self

    def get_weights(self):
        """Current (W_l, b_l) of every layer l = 1..L-1 as host arrays."""
        W, b = [], []
        for l in range(1, len(self.sizes)):
            w = np.empty((self.sizes[l - 1], self.sizes[l]), dtype=np.float32)
            v = np.empty(self.sizes[l - 1], dtype=np.float32)
            call("pcd_pc_model_get_weights", self.handle, l, w.ctypes.data, v.ctypes.data)
            W.append(w)
            b.append(v)
        return W, b


def _release_cached(key) -> None:
    """Drops a snapshot's device model from the drop-in's cache and frees it
    (W, W^T, workspaces, cached graphs); runs when the snapshot is collected."""
    hit = BatchedPcForward._cache.pop(key, None)
    if hit is not None:
        hit[1].close()


class BatchedPcForward:
    """Drop-in for the reference's static class (BatchedPcForward.cs:28-139).

    The reference transposes and uploads nothing it keeps: every call starts
    from the snapshot.  Here a snapshot's weights are uploaded once per operand
    type and kept on the device while the snapshot lives; the device model is
    freed when the snapshot is collected (a weakref finalizer), so a caller
    that makes snapshot after snapshot holds at most the live ones."""

    _cache: dict = {}

    @staticmethod
    def _model(snapshot: GenerativeSnapshot, dtype: str) -> PcDeviceModel:
        key = (id(snapshot), dtype)
        hit = BatchedPcForward._cache.get(key)
        if hit is not None and hit[0]() is snapshot:
            return hit[1]
        if hit is not None:          # an id reused by a newer object: the old model is stale
            _release_cached(key)
        m = PcDeviceModel(snapshot, dtype)
        BatchedPcForward._cache[key] = (weakref.ref(snapshot), m)
        weakref.finalize(snapshot, _release_cached, key)
        return m

    @staticmethod
    def cached_models() -> int:
        """Device models the drop-in currently holds (one per live snapshot and operand type)."""
        return len(BatchedPcForward._cache)

    @staticmethod
    def infer_get_top_batch(model: GenerativeSnapshot, inputs, inference_steps: int, mixed: bool = False,
                            dtype: str | None = None):
        """Settle every input for `inference_steps` steps; returns the top
        latent of each sample (a list of 1-D float32 arrays)."""
        if model is None:
            raise ArgumentNullException("model")
        if inputs is None:
            raise ArgumentNullException("inputs")
        if len(inputs) == 0:
            raise ArgumentException("Empty batch.")
        if inference_steps < 1:
            raise ArgumentOutOfRangeException("inferenceSteps")
        s0 = model.layer_sizes[0]
        rows = []
        for i, x in enumerate(inputs):
            x = np.asarray(x, dtype=np.float32).ravel()
            if x.size != s0:
                raise ArgumentException(f"Input {i} has {x.size} elements; the model expects {s0}.")
            rows.append(x)
        if dtype is None:
            dtype = "f16" if mixed else "f32"
        dev = BatchedPcForward._model(model, dtype)
        # rows stacked straight into the model's pinned input buffer
        top = dev._relax_top_staged(len(rows), inference_steps, lambda v: np.stack(rows, out=v))
        if top is None:
            top, _, _ = dev.relax(np.stack(rows), inference_steps)
        return list(top)
