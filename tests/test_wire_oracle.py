"""The CPU oracle of the Q8_0 hidden-state wire codec (oracle/qref_wire.c)
pinned by the reference's own tests of quantize_q8_0 / dequantize_q8_0
(src/inference/quant.rs:106-263) and by cases whose bytes follow from the
format by hand: ties of round-half-away-from-zero at scale 1, the
non-finite rules, the f16 rounding of the scale, the zero padding of a
trailing group and the byte-length rule."""
import math

import numpy as np
import pytest

from oracle import qref


def roundtrip(vals):
    vals = np.asarray(vals, np.float32)
    b = qref.wire_encode(vals)
    return b, qref.wire_decode(b, vals.size)


def test_exact_block_size_roundtrip():  # quant.rs:116-125
    vals = (np.arange(32, dtype=np.float32) - 16.0) * np.float32(0.1)
    b, rec = roundtrip(vals)
    assert b.size == 34 and rec.size == 32
    assert np.abs(vals - rec).max() < 0.01


def test_partial_trailing_block():  # quant.rs:127-137
    vals = np.arange(50, dtype=np.float32) * np.float32(0.05) - np.float32(1.0)
    b, rec = roundtrip(vals)
    assert b.size == 2 * 34 and rec.size == 50
    assert np.abs(vals - rec).max() < 0.02
    assert np.all(b[34 + 2 + 18:] == 0)  # the 14 lanes past the end are zero codes


def test_all_zeros_roundtrip():  # quant.rs:139-145
    b, rec = roundtrip(np.zeros(64, np.float32))
    assert np.all(rec == 0.0) and np.all(b == 0)


def lcg_normals(n: int) -> np.ndarray:
    """The reference's deterministic LCG + Box-Muller (quant.rs:155-172), f32."""
    seed = 0x00C0FFEE12345678
    out = np.empty(n, np.float32)
    m64 = (1 << 64) - 1

    def u01():
        nonlocal seed
        seed = (seed * 6364136223846793005 + 1442695040888963407) & m64
        return np.float32(seed >> 33) / np.float32(1 << 31)

    for i in range(n):
        u1 = u01()
        if u1 < np.float32(1e-9):
            u1 = np.float32(1e-9)
        u2 = u01()
        out[i] = np.sqrt(np.float32(-2.0) * np.log(u1)) * np.cos(np.float32(2 * math.pi) * u2)
    return out


def test_quality_gate_typical_hidden_state_distribution():  # quant.rs:148-208
    vals = lcg_normals(4096)
    for i in range(0, 4096, 100):
        vals[i] = 4.5 if i % 200 == 0 else -3.5
    _, rec = roundtrip(vals)
    assert np.abs(vals - rec).max() < 0.05
    assert np.abs(vals - rec).mean() < 0.01


def test_outlier_block_isolated():  # quant.rs:210-231
    vals = np.concatenate([np.full(32, 0.01, np.float32), np.full(32, 100.0, np.float32),
                           np.full(32, 0.01, np.float32)])
    _, rec = roundtrip(vals)
    assert np.abs(vals[:32] - rec[:32]).max() < 1e-4
    assert np.abs(vals[64:] - rec[64:]).max() < 1e-4


def test_wrong_byte_length_rejected():  # quant.rs:233-237
    with pytest.raises(ValueError):
        qref.wire_decode(np.zeros(33, np.uint8), 32)


def test_typical_hidden_state_quality():  # quant.rs:239-262
    ph = np.arange(4096, dtype=np.float32) * np.float32(0.07)
    vals = (np.sin(ph) + np.float32(0.3) * np.cos(ph * np.float32(3.1))).astype(np.float32)
    b, rec = roundtrip(vals)
    assert b.size == qref.wire_bytes(4096)
    assert 4096 * 4 / b.size > 3.5
    assert np.sqrt(np.mean((vals - rec) ** 2)) < 0.005


# ---------------------------------------------------------------------------
# bytes that follow from the format by hand
# ---------------------------------------------------------------------------
def test_scale_one_rounds_half_away_from_zero():
    # amax 127: scale = 127/127 = 1 exactly, 1/scale = 1, codes = round(v)
    vals = np.zeros(32, np.float32)
    vals[:10] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -126.5, 1.4999999, 3.0, -0.0]
    b = qref.wire_encode(vals)
    assert b[0] == 0x00 and b[1] == 0x3C  # f16 1.0 = 0x3C00, little endian
    codes = b[2:].view(np.int8)
    assert list(codes[:10]) == [127, 3, -3, 1, -1, 127, -127, 1, 3, 0]
    assert np.all(codes[10:] == 0)


def test_non_finite_values():
    vals = np.zeros(32, np.float32)
    vals[:5] = [np.inf, 1.0, np.nan, -np.inf, 2.0]
    b = qref.wire_encode(vals)
    scale = np.float32(2.0) / np.float32(127.0)  # the finite maximum only
    assert b[:2].view(np.uint16)[0] == np.float16(scale).view(np.uint16)
    codes = b[2:].view(np.int8)
    # inf * (1/scale) rounds and clamps to 127, -inf to -127, NaN codes as 0
    assert list(codes[:5]) == [127, round(1.0 / float(scale)), 0, -127, 127]
    # a block with no finite value: scale 0, 1/scale taken as 0, inf * 0 is NaN -> 0
    b2 = qref.wire_encode(np.array([np.inf, -np.inf, np.nan] + [np.nan] * 29, np.float32))
    assert np.all(b2 == 0)


def test_scale_is_stored_as_f16_and_decoded_from_it():
    vals = np.zeros(32, np.float32)
    vals[0] = np.float32(1.2345678)  # amax/127 is not an f16
    b = qref.wire_encode(vals)
    scale = np.float32(1.2345678) / np.float32(127.0)
    h = np.float16(scale)
    assert b[:2].view(np.float16)[0] == h and np.float32(h) != scale
    rec = qref.wire_decode(b, 32)
    assert rec[0] == np.float32(127) * np.float32(h)  # the f16 scale, not the f32 one


def test_byte_lengths():
    assert [qref.wire_bytes(n) for n in (0, 1, 31, 32, 33, 64, 65)] == [0, 34, 34, 34, 68, 68, 102]
    assert qref.wire_bytes(2 ** 62) == (2 ** 62 // 32) * 34
    assert qref.wire_bytes(2 ** 63 - 1) == -1  # ceil(n/32)*34 overflows: rejected, never wrapped
