"""LayerSerializer records, restated (TEST INFRASTRUCTURE ONLY).

A CPU restatement of the reference's per-layer record format and its weight
codecs (PredicitiveCoding/Model/LayerSerializer.cs), used by tests/ to write
records the way the reference persists them and to say what loading one must
give.  Only tests/ may import it; the product path parses records itself
(pcd_pc_model_load_record).

Layout (LayerSerializer.cs:8-41), little-endian:
    0  int32 Size      4  int32 LowerSize   8  float32 Precision
   12  float32 WeightDecay  16 StateLearningRate  20 WeightLearningRate
   24  byte IsClamped  25  byte flags (1 diag precision, 2 prior mean,
       4 Half weights, 8 bfloat16 weights, 16 int8 affine weights)  26 pad[2]
   28  Mu [Size] f32, PredictionError [Size] f32
   if LowerSize > 0: weights [LowerSize x Size] in the stored format,
       then Bias, PreActivation, Prediction [LowerSize] f32 each
"""
from __future__ import annotations

import struct

import numpy as np

from . import pc_oracle

FLOAT32, HALF, BF16, INT8 = "float32", "half", "bf16", "int8"
_FLAG = {FLOAT32: 0, HALF: 4, BF16: 8, INT8: 16}
HEADER = 28   # FixedHeaderBytes, LayerSerializer.cs:45


def byte_length(size: int, lower: int, fmt: str = FLOAT32) -> int:
    """ComputeByteLength (LayerSerializer.cs:208-228), no diagonal/prior."""
    n = HEADER + size * 8
    if lower > 0:
        n += {FLOAT32: lower * size * 4, HALF: lower * size * 2, BF16: lower * size * 2,
              INT8: lower * 4 + lower + lower * size}[fmt]
        n += lower * 3 * 4
    return n


def int8_quantize(w: np.ndarray):
    """WriteInt8Weights (LayerSerializer.cs:241-285): per-row scale s and zero
    point z, codes q = clamp(round(w/s) + z, -128, 127); all in float32, with
    MathF.Round's round-half-to-even."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    scales = np.empty(rows, np.float32)
    zeros = np.empty(rows, np.int8)
    codes = np.empty((rows, cols), np.int8)
    for r in range(rows):
        lo = np.float32(w[r].min())
        hi = np.float32(w[r].max())
        if np.float32(hi - lo) < np.float32(1e-12):
            s = np.float32(max(abs(lo), np.float32(1e-12))) / np.float32(127.0)
            z = 0
        else:
            s = np.float32(hi - lo) / np.float32(255.0)
            z = int(np.clip(int(np.rint(np.float32(-lo) / s)) - 128, -128, 127))
        scales[r] = s
        zeros[r] = z
        q = np.rint(w[r] / s).astype(np.int64) + z
        codes[r] = np.clip(q, -128, 127).astype(np.int8)
    return scales, zeros, codes


def int8_dequantize(scales, zeros, codes) -> np.ndarray:
    """ReadInt8Weights (LayerSerializer.cs:288-303): w = (q - z) * s."""
    q = codes.astype(np.int32) - zeros.astype(np.int32)[:, None]
    return (q.astype(np.float32) * scales[:, None].astype(np.float32)).astype(np.float32)


def serialize(size: int, lower: int, precision: float, W=None, b=None, fmt: str = FLOAT32,
              weight_decay: float = 0.0, state_lr: float = 0.1, weight_lr: float = 0.01) -> bytes:
    """LayerSerializer.Serialize (:73-143) for a layer without diagonal precision
    or prior; Mu, PredictionError, PreActivation and Prediction are written zero."""
    if lower == 0:
        fmt = FLOAT32
    out = bytearray()
    out += struct.pack("<iiffff", size, lower, precision, weight_decay, state_lr, weight_lr)
    out += bytes([0, _FLAG[fmt], 0, 0])
    out += np.zeros(2 * size, np.float32).tobytes()
    if lower > 0:
        W = np.ascontiguousarray(W, dtype=np.float32).reshape(lower, size)
        if fmt == HALF:
            out += W.astype(np.float16).tobytes()                # TensorUtils.ToHalf, round to nearest even
        elif fmt == BF16:
            out += pc_oracle.bf16_bits(W).tobytes()              # TensorUtils.FloatToBf16Bits
        elif fmt == INT8:
            s, z, q = int8_quantize(W)
            out += s.tobytes() + z.tobytes() + q.tobytes()
        else:
            out += W.tobytes()
        out += np.ascontiguousarray(b, dtype=np.float32).tobytes()
        out += np.zeros(2 * lower, np.float32).tobytes()
    assert len(out) == byte_length(size, lower, fmt)
    return bytes(out)


def deserialize(record: bytes):
    """LayerSerializer.Deserialize (:147-205) of the fields a settling needs:
    returns (size, lower, precision, fmt, W [lower x size] float32 widened as the
    reference widens it into its masters, b)."""
    size, lower = struct.unpack_from("<ii", record, 0)
    precision = struct.unpack_from("<f", record, 8)[0]
    flags = record[25]
    fmt = {0: FLOAT32, 4: HALF, 8: BF16, 16: INT8}[flags & 28]
    pos = HEADER + size * 8
    W = b = None
    if lower > 0:
        n = lower * size
        if fmt == FLOAT32:
            W = np.frombuffer(record, np.float32, n, pos).reshape(lower, size).copy()
            pos += n * 4
        elif fmt == HALF:
            W = np.frombuffer(record, np.float16, n, pos).astype(np.float32).reshape(lower, size)
            pos += n * 2
        elif fmt == BF16:
            bits = np.frombuffer(record, np.uint16, n, pos).astype(np.uint32) << 16
            W = bits.view(np.float32).reshape(lower, size).copy()
            pos += n * 2
        else:
            s = np.frombuffer(record, np.float32, lower, pos)
            z = np.frombuffer(record, np.int8, lower, pos + lower * 4)
            q = np.frombuffer(record, np.int8, n, pos + lower * 5).reshape(lower, size)
            W = int8_dequantize(s, z, q)
            pos += lower * 5 + n
        b = np.frombuffer(record, np.float32, lower, pos).copy()
    return size, lower, precision, fmt, W, b
