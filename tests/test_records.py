"""Pins of the record restatement (oracle/records.py) against the layout table
and the behaviours the reference's own tests assert (MixedSub16Tests.cs), plus
hand-worked int8 quantizer cases."""
import struct

import numpy as np
import pytest

from oracle import records as rec
from tests.netgen import make_net


def test_float32_record_layout_by_hand():
    # LayerSerializer.cs:12-36, written field by field
    W = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], np.float32)
    b = np.array([0.5, -0.5], np.float32)
    want = (struct.pack("<i", 3) + struct.pack("<i", 2) + struct.pack("<f", 1.25) + struct.pack("<f", 0.0)
            + struct.pack("<f", 0.1) + struct.pack("<f", 0.01) + b"\x00" + b"\x00" + b"\x00\x00"
            + b"\x00" * 24                          # Mu[3] + PredictionError[3]
            + W.tobytes() + b.tobytes() + b"\x00" * 16)
    got = rec.serialize(3, 2, 1.25, W, b)
    assert got == want and len(got) == rec.byte_length(3, 2)
    size, lower, prec, fmt, W2, b2 = rec.deserialize(want)
    assert (size, lower, prec, fmt) == (3, 2, 1.25, rec.FLOAT32)
    assert np.array_equal(W2, W) and np.array_equal(b2, b)


def test_layer_zero_record_has_no_weights():
    r = rec.serialize(5, 0, 0.75)
    assert len(r) == 28 + 40
    assert rec.deserialize(r)[:4] == (5, 0, 0.75, rec.FLOAT32)


def test_int8_known_answer_by_hand():
    # row [-1, 0, 1, 2.5]: s = 3.5/255, z = round(1/s) - 128 = 73 - 128 = -55,
    # q = round(w/s) + z = [-128, -55, 18, 127]
    w = np.array([[-1.0, 0.0, 1.0, 2.5]], np.float32)
    s, z, q = rec.int8_quantize(w)
    s_hand = np.float32(3.5) / np.float32(255.0)
    assert s[0] == s_hand and z[0] == -55
    assert list(q[0]) == [-128, -55, 18, 127]
    back = rec.int8_dequantize(s, z, q)
    assert np.allclose(back[0], (np.array([-128, -55, 18, 127]) + 55) * float(s_hand), rtol=0, atol=1e-7)


def test_int8_constant_row_and_round_half_even():
    s, z, q = rec.int8_quantize(np.array([[0.3, 0.3, 0.3]], np.float32))
    assert z[0] == 0 and s[0] == np.float32(0.3) / np.float32(127.0) and list(q[0]) == [127, 127, 127]
    # a value exactly halfway between two codes rounds to the even code (MathF.Round)
    w = np.array([[0.0, 2.55]], np.float32)              # s = 0.01, z = -128
    s, z, q = rec.int8_quantize(w)
    assert z[0] == -128
    half = np.float32(0.5) * s[0]                         # w/s = 0.5 exactly
    q2 = np.rint(np.float32(half) / s[0])
    assert q2 == 0.0


def test_bf16_record_matches_reference_test():
    # MixedSub16Tests.cs:58-84: two bytes per weight, |w~ - w| <= |w|/128, idempotent
    W, b, _ = make_net([3, 4], seed=5, bias_scale=0.2)
    full = rec.serialize(4, 3, 1.0, W[0], b[0])
    bf = rec.serialize(4, 3, 1.0, W[0], b[0], fmt=rec.BF16)
    assert len(full) - len(bf) == 3 * 4 * 2
    _, _, _, fmt, Wb, bb = rec.deserialize(bf)
    assert fmt == rec.BF16 and np.array_equal(bb, b[0])
    assert np.all(np.abs(Wb - W[0]) <= np.abs(W[0]) / 128 + 1e-12)
    again = rec.deserialize(rec.serialize(4, 3, 1.0, Wb, bb, fmt=rec.BF16))[4]
    assert np.array_equal(again, Wb)


def test_int8_record_matches_reference_test():
    # MixedSub16Tests.cs:86-122: scales + zero points + codes, error <= (max-min)/255 / 2 + 1e-6 per row
    W, b, _ = make_net([6, 9], seed=6, bias_scale=0.2)
    w = W[0]
    full = rec.serialize(9, 6, 1.0, w, b[0])
    i8 = rec.serialize(9, 6, 1.0, w, b[0], fmt=rec.INT8)
    assert len(full) - len(i8) == 6 * 9 * 4 - (6 * 4 + 6 + 6 * 9)
    _, _, _, fmt, Wq, _ = rec.deserialize(i8)
    assert fmt == rec.INT8
    for r in range(6):
        bound = (w[r].max() - w[r].min()) / 255.0 * 0.5 + 1e-6
        assert np.all(np.abs(Wq[r] - w[r]) <= bound)


def test_half_record_widens_exactly():
    W, b, _ = make_net([5, 7], seed=7)
    h = rec.serialize(7, 5, 1.0, W[0], b[0], fmt=rec.HALF)
    _, _, _, fmt, Wh, _ = rec.deserialize(h)
    assert fmt == rec.HALF
    assert np.array_equal(Wh, W[0].astype(np.float16).astype(np.float32))
