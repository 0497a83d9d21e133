"""Pins the CPU oracle (oracle/) to the reference's own known answers.

Every check here is one the reference's tests make (cited per test), or one
the mathematics fixes (IEEE binary16 against numpy's independent
conversion, integer sums against brute force in int64). A plausible mistake
in the oracle — a dropped term, a wrong sign, index or nibble order, a
changed summation order — fails at least one of them.
"""
import numpy as np
import pytest

from oracle import qref
from inputs import (StdRng, fnv1a, ggml_like_vector, iq4_inputs, lcg_noise, mxfp4_inputs,
                    random_tensors, round3, rust_round, get_test_vector2)

H = lambda s: int(s, 16)  # noqa: E731


# ---------------------------------------------------------------------------
# f16 conversion (half 2.7.1 = IEEE binary16 RNE): against numpy.float16.
# ---------------------------------------------------------------------------
def test_f16_to_f32_all_65536_codes():
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([qref.f16_bits_to_f32(int(c)) for c in codes], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_f32_to_f16_rne_boundaries():
    rng = np.random.default_rng(7)
    # every f16 value, its midpoints to the next value, and a ulp either side
    f16 = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    nxt = np.arange(1, 0x7C01, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((f16.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    cases = np.concatenate([f16, mids, np.nextafter(mids, np.float32(np.inf)),
                            np.nextafter(mids, np.float32(0)),
                            rng.standard_normal(20000).astype(np.float32) * 30,
                            np.float32([65504, 65519.99, 65520, 1e-8, 3e-8, 6e-8, 1e30])])
    cases = np.concatenate([cases, -cases])
    with np.errstate(over="ignore"):
        want = cases.astype(np.float16).view(np.uint16)
    got = np.array([qref.f32_to_f16_bits(float(c)) for c in cases], dtype=np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(cases[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


# ---------------------------------------------------------------------------
# MXFP4: src/inference/mod.rs:1466-1531
# ---------------------------------------------------------------------------
def test_mxfp4_reads_multiplies_and_quantizes_as_llama_cpp_does(kats):
    k = kats["mxfp4"]
    x, y, src = mxfp4_inputs()
    deq = qref.to_float(qref.MXFP4, x, 9 * 32)
    assert fnv1a(deq.tobytes()) == H(k["dequant_fnv1a"])
    assert int(deq.view(np.uint32)[0]) == H(k["dequant_first_bits"])
    q = qref.from_float(qref.MXFP4, src)
    assert q.size == 6 * 17
    assert fnv1a(q.tobytes()) == H(k["quantized_fnv1a"])
    want8, want9 = np.uint32(H(k["dot8_bits"])).view(np.float32), np.uint32(H(k["dot9_bits"])).view(np.float32)
    dot8 = qref.vec_dot(qref.MXFP4, 8 * 32, x[: 8 * 17], y[: 8 * 34])
    dot9 = qref.vec_dot(qref.MXFP4, 9 * 32, x, y)
    # AVX2 order: bit for bit (the odd ninth block by the scalar rule)
    assert (dot8.view(np.uint32), dot9.view(np.uint32)) == (H(k["dot8_bits"]), H(k["dot9_bits"]))
    for got, want in [(dot8, want8), (dot9, want9),
                      (qref.vec_dot_unopt(qref.MXFP4, 256, x[: 8 * 17], y[: 8 * 34]), want8),
                      (qref.vec_dot_unopt(qref.MXFP4, 288, x, y), want9)]:
        assert abs(got - want) <= 1e-5 * abs(want)


def test_mxfp4_nibble_order(kats):
    """src/inference/mod.rs:1513-1530: low nibble of byte j is element j."""
    table = kats["mxfp4"]["nibble_table"]
    blk = np.array([127] + [j | ((15 - j) << 4) for j in range(16)], dtype=np.uint8)
    out = qref.to_float(qref.MXFP4, blk, 32)
    for j in range(16):
        assert out[j] == table[j] * 0.5
        assert out[j + 16] == table[15 - j] * 0.5


# ---------------------------------------------------------------------------
# IQ4_NL: src/inference/mod.rs:1767-1863
# ---------------------------------------------------------------------------
def test_iq4_nl_reads_multiplies_and_quantizes_as_llama_cpp_does(kats):
    k = kats["iq4_nl"]
    nl, q8, nl_src = iq4_inputs()
    deq = qref.to_float(qref.IQ4_NL, nl, 9 * 32)
    assert fnv1a(deq.tobytes()) == H(k["dequant_fnv1a"])
    for nb, key in [(8, "dot8_bits"), (9, "dot9_bits")]:
        want_bits = H(k[key])
        want = np.uint32(want_bits).view(np.float32)
        got = qref.vec_dot(qref.IQ4_NL, nb * 32, nl[: nb * 18], q8[: nb * 34])
        assert int(got.view(np.uint32)) == want_bits
        unopt = qref.vec_dot_unopt(qref.IQ4_NL, nb * 32, nl[: nb * 18], q8[: nb * 34])
        assert abs(unopt - want) <= 1e-5 * abs(want)
    q = qref.from_float(qref.IQ4_NL, nl_src)
    assert fnv1a(q.tobytes()) == H(k["quantized_fnv1a"])


def test_iq4_nl_nibble_order(kats):
    table = kats["iq4_nl"]["nibble_table"]
    blk = np.array([0x00, 0x3C] + [j | ((15 - j) << 4) for j in range(16)], dtype=np.uint8)
    out = qref.to_float(qref.IQ4_NL, blk, 32)
    for j in range(16):
        assert out[j] == table[j]
        assert out[j + 16] == table[15 - j]


# ---------------------------------------------------------------------------
# Q8_K: src/inference/mod.rs:1887-1907 (largest activation at +-127)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("big", [1.0, -1.0])
def test_q8k_writes_its_largest_activation_at_127(big):
    xs = np.full(256, 0.25, dtype=np.float32)
    xs[7] = big
    xs[8] = -0.75
    raw = qref.from_float(qref.Q8_K, xs)
    d = raw[0:4].view(np.float32)[0]
    qs = raw[4:260].view(np.int8)
    assert qs[7] == -127
    assert np.all(qs != -128)
    assert d == np.float32(-big) / np.float32(127.0)
    assert qs[8] == int(rust_round(np.float32(127.0) * np.float32(0.75) * np.sign(big)))
    bsums = raw[260:292].view(np.int16)
    assert np.array_equal(bsums, qs.astype(np.int64).reshape(16, 16).sum(1))


def test_q8k_activation_codes_brute_force():
    """Closed form of BlockQ8K::from_float (Q/k_quants.rs:2882-2927), checked in
    float64 where every f32 step is exact or rounded once: codes within +-127,
    reconstruction within half a step, bsums the exact group sums, and the
    first largest-|x| element always written at -127 (ties keep the first)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(256 * 64).astype(np.float32)
    x[256 * 5 + 17] = 9.0
    x[256 * 5 + 200] = -9.0   # a tie in |x|: the first (positive) one sets the sign
    x[256 * 9: 256 * 10] = 0  # an all-zero block: d = 0, codes 0
    raw = qref.from_float(qref.Q8_K, x).reshape(64, 292)
    d = raw[:, :4].copy().view(np.float32).ravel()
    qs = raw[:, 4:260].view(np.int8).astype(np.int64)
    bs = raw[:, 260:].copy().view(np.int16).astype(np.int64)
    xb = x.reshape(64, 256).astype(np.float64)
    assert d[9] == 0 and not qs[9].any()
    for b in range(64):
        if b == 9:
            continue
        assert np.array_equal(bs[b], qs[b].reshape(16, 16).sum(1))
        first = int(np.argmax(np.abs(xb[b])))
        assert qs[b][first] == -127
        assert np.all(np.abs(qs[b]) <= 127)
        assert np.all(np.abs(qs[b] * np.float64(d[b]) - xb[b]) <= abs(d[b]) * 0.50001)
    assert np.sign(d[5]) == -1  # max = +9.0 -> iscale < 0 -> d < 0


def test_q8_0_activation_codes_brute_force():
    """BlockQ8_0::from_float (Q/k_quants.rs:1240-1269): d = f16(amax/127),
    codes = round(x / d_unrounded), |q| <= 127."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal(32 * 200).astype(np.float32) * np.float32(3)
    x[32 * 7: 32 * 8] = 0
    raw = qref.from_float(qref.Q8_0, x).reshape(200, 34)
    dh = raw[:, :2].copy().view(np.float16).ravel()
    qs = raw[:, 2:].view(np.int8).astype(np.int64)
    xb = x.reshape(200, 32).astype(np.float64)
    amax = np.abs(x.reshape(200, 32)).max(1)
    d32 = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(dh, d32.astype(np.float16))
    assert not qs[7].any()
    for b in range(200):
        if b == 7:
            continue
        assert np.all(np.abs(qs[b]) <= 127)
        assert np.all(np.abs(qs[b] * np.float64(d32[b]) - xb[b]) <= d32[b] * 0.5000001)
        assert 127 in np.abs(qs[b])


@pytest.fixture
def q8k_scale_128():
    """SWARMLLM_Q8K_SCALE=128 (Q/k_quants.rs:145-152): candle's Q8_K scale before
    the #404 patch, which candle's own QMatMul KATs were recorded with."""
    import ctypes
    L = qref.lib()
    L.qref_set_q8k_scale.argtypes = [ctypes.c_float]
    L.qref_set_q8k_scale(128.0)
    yield
    L.qref_set_q8k_scale(127.0)


# ---------------------------------------------------------------------------
# Spot dequant values and error bounds: tests/quantized_tests.rs:450-471, 765-931
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name,qtype", [("q4_k", qref.Q4_K), ("q6_k", qref.Q6_K), ("q8_k", qref.Q8_K)])
def test_spot_dequant_values(kats, name, qtype, request):
    if qtype == qref.Q8_K:  # recorded before the #404 Q8_K scale patch
        request.getfixturevalue("q8k_scale_128")
    s = kats["spot_dequant"]
    src = get_test_vector2(0.5, 1024)
    assert np.array_equal(src[s["indices"]], np.float32(s["src"]))
    dst = qref.to_float(qtype, qref.from_float(qtype, src), 1024)
    assert np.all(np.abs(dst - src) < s[name]["tol"])
    assert np.array_equal(np.float32(round3([dst[i] for i in s["indices"]])), np.float32(s[name]["dst"]))
    big = get_test_vector2(128.0, 1024)
    dbig = qref.to_float(qtype, qref.from_float(qtype, big), 1024)
    assert np.all(np.abs(dbig - big) < s[name]["tol_big"])


@pytest.mark.parametrize("qtype", [qref.Q4_K, qref.Q6_K, qref.Q8_K, qref.Q8_0, qref.Q4_0])
def test_quantization_rmse(kats, qtype):
    src = ggml_like_vector(0.0)
    dst = qref.to_float(qtype, qref.from_float(qtype, src), src.size)
    rmse = np.sqrt(np.sum((src.astype(np.float64) - dst) ** 2)) / src.size
    assert rmse <= kats["quantization_rmse"]["max_error"]


@pytest.mark.parametrize("name,qtype", [("q4_k", qref.Q4_K), ("q6_k", qref.Q6_K), ("q8_0", qref.Q8_0),
                                        ("q4_0", qref.Q4_0)])
def test_matmul_error(kats, name, qtype):
    """ggml_matmul_error_test: tests/quantized_tests.rs:1045-1110."""
    cfg = kats["matmul_error"]
    n = 32 * 128
    cases = [(ggml_like_vector(0.0), ggml_like_vector(1.0), 1.0),
             (np.arange(n, dtype=np.float32) / np.float32(n), np.arange(n, dtype=np.float32) / np.float32(n), 2.0)]
    for a, b, err_m in cases:
        aq = qref.from_float(qtype, a)
        bq = qref.from_float(qref.VEC_DOT[qtype], b)
        r = qref.vec_dot(qtype, n, aq, bq)
        ru = qref.vec_dot_unopt(qtype, n, aq, bq)
        assert abs(r - ru) / n <= 1e-6
        rm = qref.matmul(qtype, b.reshape(1, n), aq, 1)[0, 0]
        assert abs(rm - r) / n <= 1e-6
        ref = np.float32(0)
        for ai, bi in zip(a, b):
            ref = np.float32(ref + ai * bi)
        for v in (r, rm):
            err = abs(float(v) - float(ref)) / n
            assert np.isfinite(err) and err <= cfg["max_dot_error"]
            assert err - cfg["leniency"] <= cfg["ggml_error"][name] * err_m


# ---------------------------------------------------------------------------
# Q4_0 closed-form matmul: tests/quantized_tests.rs:91-221 (CPU arm)
# ---------------------------------------------------------------------------
def test_q4_0_closed_form_matmul(kats):
    m, k, n = 3, 64, 4
    lhs = np.arange(m * k, dtype=np.float32).reshape(m, k)
    rhs = np.arange(k * n, dtype=np.float32)
    w = qref.from_float(qref.Q4_0, rhs)
    got = rust_round(qref.matmul(qref.Q4_0, lhs, w, n).ravel())
    assert got.tolist() == kats["q4_0_matmul"]["pos"]
    lhs = (np.arange(m * k, dtype=np.float32) - np.float32(m * k / 2)).reshape(m, k)
    rhs = np.arange(k * n, dtype=np.float32) - np.float32(k * n) / np.float32(3)
    w = qref.from_float(qref.Q4_0, rhs)
    got = rust_round(qref.matmul(qref.Q4_0, lhs, w, n).ravel())
    assert got.tolist() == kats["q4_0_matmul"]["neg"]


# ---------------------------------------------------------------------------
# Seeded QMatMul KATs: tests/quantized_tests.rs:1127-1148, 1301-1377
# ---------------------------------------------------------------------------
def test_stdrng_restatement_reproduces_the_f32_kat(kats):
    c = kats["qmatmul_chacha"]
    lhs, rhs = random_tensors(c["m"], c["k"], c["n"], c["seed"])
    mm = (lhs.astype(np.float64) @ rhs.astype(np.float64).T).ravel()
    mn = c["m"] * c["n"]
    assert round3([mm[0], mm[mn // 3], mm[mn * 2 // 3], mm[mn - 1]]) == c["f32"]


@pytest.mark.parametrize("name,qtype", [("q4_k", qref.Q4_K), ("q6_k", qref.Q6_K)])
def test_qmatmul_kat(kats, name, qtype, q8k_scale_128):
    """Pins Q4_K/Q6_K from_float (make_qkx1_quants / make_qx_quants), the Q8_K
    quantizer and the several-row dots (m = 11: two 4-row passes + a 3-row tail)."""
    c = kats["qmatmul_chacha"]
    lhs, rhs = random_tensors(c["m"], c["k"], c["n"], c["seed"])
    w = qref.from_float(qtype, rhs)
    mm = qref.matmul(qtype, lhs, w, c["n"]).ravel()
    mn = c["m"] * c["n"]
    assert round3([mm[0], mm[mn // 3], mm[mn * 2 // 3], mm[mn - 1]]) == c[name]


@pytest.mark.parametrize("qtype", [qref.Q4_K, qref.Q6_K])
def test_qmatmul_kat_differs_at_the_patched_scale(kats, qtype):
    """At the default 127 scale the same product moves (the #404 patch is live):
    the knob above is what makes the KAT match, not a loose comparison."""
    c = kats["qmatmul_chacha"]
    lhs, rhs = random_tensors(c["m"], c["k"], c["n"], c["seed"])
    mm = qref.matmul(qtype, lhs, qref.from_float(qtype, rhs), c["n"]).ravel()
    mn = c["m"] * c["n"]
    name = "q4_k" if qtype == qref.Q4_K else "q6_k"
    assert round3([mm[0], mm[mn // 3], mm[mn * 2 // 3], mm[mn - 1]]) != c[name]


# ---------------------------------------------------------------------------
# Driver exactness: src/inference/mod.rs:1266-1385
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qtype", [qref.Q4_K, qref.Q6_K, qref.Q8_0, qref.Q4_0, qref.MXFP4, qref.IQ4_NL])
def test_tiled_and_several_row_kernels_are_bit_identical_to_per_row(qtype):
    k, n = 512, 96
    noise = lcg_noise(0x9E3779B97F4A7C15)
    w = qref.from_float(qtype, noise(n * k))
    for m in [1, 2, 3, 4, 5, 7, 8, 9, 13, 130]:
        lhs = noise(m * k).reshape(m, k)
        got = qref.matmul(qtype, lhs, w, n)
        want = qref.matmul_upstream(qtype, lhs, w, n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (qtype, m)


def test_several_row_kernel_matches_per_row_loop():
    rng = np.random.default_rng(11)
    for qtype in (qref.Q4_K, qref.Q6_K, qref.Q8_0, qref.Q4_0):
        k = 1024
        w = qref.from_float(qtype, rng.standard_normal(k).astype(np.float32))
        for rows in (1, 2, 3, 4, 5, 6, 7, 11):
            xq = qref.quantize_rows(qtype, rng.standard_normal((rows, k)).astype(np.float32))
            a = np.empty(rows, np.float32)
            b = np.empty(rows, np.float32)
            L = qref.lib()
            L.qref_vec_dot_rows(qtype, k, w.ctypes.data, xq.ctypes.data, rows, a.ctypes.data, 0)
            L.qref_vec_dot_rows(qtype, k, w.ctypes.data, xq.ctypes.data, rows, b.ctypes.data, 1)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (qtype, rows)


@pytest.mark.parametrize("qtype", [qref.Q8_0, qref.Q4_0, qref.MXFP4, qref.IQ4_NL])
def test_32_value_dots_agree_with_the_scalar_loop(qtype):
    k = 896
    noise = lcg_noise(0x2545F4914F6CDD1D)
    for trial in range(64):
        w = noise(k)
        a = (noise(k) + np.float32(0.3 if trial % 2 == 0 else 0.0)).astype(np.float32)
        col = qref.from_float(qtype, w)
        row = qref.from_float(qref.VEC_DOT[qtype], a)
        got = qref.vec_dot(qtype, k, col, row)
        want = qref.vec_dot_unopt(qtype, k, col, row)
        assert abs(got - want) <= 1e-4 * (1.0 + abs(want))


@pytest.mark.parametrize("qtype", [qref.Q4_K, qref.Q6_K])
def test_k_quant_dots_agree_with_the_scalar_loop(qtype):
    rng = np.random.default_rng(5)
    k = 4096
    for _ in range(16):
        col = qref.from_float(qtype, rng.standard_normal(k).astype(np.float32) * np.float32(0.02))
        row = qref.from_float(qref.Q8_K, rng.standard_normal(k).astype(np.float32))
        got = qref.vec_dot(qtype, k, col, row)
        want = qref.vec_dot_unopt(qtype, k, col, row)
        assert abs(got - want) <= 1e-5 * (1e-3 + abs(want)) + 1e-6


@pytest.mark.parametrize("qtype", [qref.Q4_K, qref.Q6_K, qref.Q8_0, qref.MXFP4, qref.IQ4_NL])
def test_dot_equals_exact_dequantized_product(qtype):
    """The integer core of every dot, brute force: the dot of the dequantized
    weight with the dequantized activation (float64) matches the kernel to
    f32 rounding. A wrong index, sign, nibble or scale misses by far more."""
    rng = np.random.default_rng(9)
    k = 2048
    for _ in range(8):
        w = rng.standard_normal(k).astype(np.float32) * np.float32(0.02)
        a = rng.standard_normal(k).astype(np.float32)
        col = qref.from_float(qtype, w)
        vt = qref.VEC_DOT[qtype]
        row = qref.from_float(vt, a)
        exact = float(np.dot(qref.to_float(qtype, col, k).astype(np.float64),
                             qref.to_float(vt, row, k).astype(np.float64)))
        scale = float(np.linalg.norm(qref.to_float(qtype, col, k)) * np.linalg.norm(a))
        for f in (qref.vec_dot, qref.vec_dot_unopt):
            assert abs(float(f(qtype, k, col, row)) - exact) <= 1e-5 * scale
