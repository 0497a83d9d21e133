"""The CPU oracle of the gated activations act(gate) * up (oracle/qref_glu.c)
pinned by the reference's own test vectors and by closed forms:

- SwigluOai: the reference's test input (fast_math.rs:508-560, edge values
  either side of both clamps and 4093 xorshift pairs) and the FNV-1a digest
  of llama.cpp's output on it that the reference asserts on glibc;
- SiLU and GELU: float64 evaluations of their formulas, the limits where
  exp / tanh saturate, zeros, signed zeros and NaN.
"""
import numpy as np
import pytest

from oracle import qref


def swiglu_inputs():
    """The reference's inputs (fast_math.rs:512-533): eleven edge values, then
    xorshift32 pairs mapped to [-10, 10] in f32."""
    gate = [-90.0, -7.5, -7.0, -1.0, -0.0, 0.0, 0.3, 6.99, 7.0, 7.01, 50.0]
    up = [-50.0, -7.01, -7.0, -1.0, 0.0, -0.0, 0.7, 6.99, 7.0, 7.01, 90.0]
    gate = [np.float32(v) for v in gate]
    up = [np.float32(v) for v in up]
    s = 0x9E3779B9
    m = 0xFFFFFFFF

    def step(s):
        s ^= (s << 13) & m
        s ^= s >> 17
        s ^= (s << 5) & m
        return s

    for _ in range(4093):
        s = step(s)
        gate.append(np.float32(s % 40001) / np.float32(2000.0) - np.float32(10.0))
        s = step(s)
        up.append(np.float32(s % 40001) / np.float32(2000.0) - np.float32(10.0))
    return np.array(gate, np.float32), np.array(up, np.float32)


def fnv1a64(b: bytes) -> int:
    h = 0xCBF29CE484222325
    for c in b:
        h = ((h ^ c) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_swiglu_oai_matches_llama_cpps_output_digest():  # fast_math.rs:540-556
    g, u = swiglu_inputs()
    assert (g > 7.0).any() and (u < -7.0).any()
    out = qref.glu("swiglu_oai", g, u)
    assert fnv1a64(out.astype("<f4").tobytes()) == 0xA594237E1C52159C


def test_swiglu_oai_nan_and_clamps():
    g = np.array([np.nan, 1.0, 8.0, 7.0, -3.0], np.float32)
    u = np.array([1.0, np.nan, 100.0, -100.0, 0.5], np.float32)
    out = qref.glu("swiglu_oai", g, u)
    assert np.isnan(out[0]) and np.isnan(out[1])  # std::min(NaN, limit) and clamp keep NaN
    # the gate is clamped from above only; up both ways, then lifted by one
    x = np.float32(7.0)
    assert out[2] == x / (np.float32(1) + np.exp(np.float32(1.702) * -x)) * np.float32(8.0)
    assert out[3] == x / (np.float32(1) + np.exp(np.float32(1.702) * -x)) * np.float32(-6.0)
    assert out[4] < 0  # a negative gate is not clamped from below


def test_silu_closed_form_and_limits():
    rng = np.random.default_rng(0)
    g = (rng.standard_normal(20000) * 3).astype(np.float32)
    u = rng.standard_normal(20000).astype(np.float32)
    out = qref.glu("silu", g, u).astype(np.float64)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    want = gd / (1.0 + np.exp(-gd)) * ud
    assert np.max(np.abs(out - want) / np.maximum(np.abs(want), 1e-30)) < 4e-7
    s = qref.glu("silu", np.array([0.0, 100.0, -100.0, -0.0, np.nan], np.float32),
                 np.array([3.0, 2.0, 1.0, 1.0, 1.0], np.float32))
    assert s[0] == 0.0 and s[1] == 200.0  # exp(-100) underflows: g / 1 * u
    assert s[2] == 0.0 and np.signbit(s[2])  # exp(100) is inf: -100 / inf = -0
    assert s[3] == 0.0 and np.isnan(s[4])


def test_gelu_tanh_form():
    rng = np.random.default_rng(1)
    g = (rng.standard_normal(20000) * 3).astype(np.float32)
    u = rng.standard_normal(20000).astype(np.float32)
    out = qref.glu("gelu", g, u).astype(np.float64)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    want = 0.5 * gd * (1.0 + np.tanh(0.7978846 * gd * (1.0 + 0.044715 * gd * gd))) * ud
    # relative to the value, plus the f32 cancellation of 1 + tanh near -1
    # (about an ulp of 1 times 0.5 |v u|), which the reference's f32 form has too
    assert np.all(np.abs(out - want) <= 2e-5 * np.abs(want) + 2e-7 * np.abs(gd * ud))
    # far from zero the tanh form is v for v > 0 and 0 for v < 0
    s = qref.glu("gelu", np.array([0.0, 20.0, -20.0], np.float32), np.ones(3, np.float32))
    assert s[0] == 0.0 and s[1] == 20.0 and s[2] == 0.0


@pytest.mark.parametrize("act", ["silu", "swiglu_oai", "gelu"])
def test_glu_rejects_mismatched_shapes(act):
    with pytest.raises(ValueError):
        qref.glu(act, np.zeros(3, np.float32), np.zeros(4, np.float32))
