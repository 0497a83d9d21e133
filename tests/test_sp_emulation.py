"""The CPU emulation of the approximate-operand kernels (tests/sp_emulation.py)
pinned on the CPU: its block parsing reproduces the oracle's product when
the operands are made exact (a wrong nibble order, scale index or sign
fails this), and its rounded operands stay inside the 2e-3 bound on weights
with one sub-block per super-block 10-100x the rest, on C3's x20-outlier
activations and on activations concentrated on the small sub-blocks, while
differing from the exact product (the rounding is really modelled)."""
import numpy as np
import pytest

import sp_emulation as emu
from helpers import TOL_GEMM, normalised_error
from oracle import qref

N, K, M = 48, 2048, 12


def case(fmt, factor, acts, seed):
    rng = np.random.default_rng(seed)
    unit = 32 if fmt == qref.Q4_K else 16
    w, big = emu.skewed_weights(rng, N, K, unit, factor)
    x = emu.concentrated_activations(rng, M, K, big, unit) if acts == "small" else emu.outlier_activations(rng, M, K)
    wq = qref.from_float(fmt, w)
    xq = qref.quantize_rows(fmt, x)
    want = qref.matmul(fmt, x, wq, N).astype(np.float64)
    wdeq = qref.to_float(fmt, wq, N * K).reshape(N, K)
    return wq, xq, x, want, wdeq


@pytest.mark.parametrize("factor", [1, 10, 100])
@pytest.mark.parametrize("acts", ["outliers", "small"])
def test_q4k_emulation(factor, acts):
    wq, xq, x, want, wdeq = case(qref.Q4_K, factor, acts, 1000 + factor)
    exact = emu.q4k_single_pass(wq, N, K, xq, M, mode="exact")
    assert normalised_error(exact, want, wdeq, x) < 1e-6
    approx = emu.q4k_single_pass(wq, N, K, xq, M)
    err = normalised_error(approx, want, wdeq, x)
    assert 1e-6 < err <= TOL_GEMM, err


@pytest.mark.parametrize("factor", [1, 10, 100])
@pytest.mark.parametrize("acts", ["outliers", "small"])
@pytest.mark.parametrize("form", ["gemm", "few_rows"])
def test_q6k_emulation(factor, acts, form):
    wq, xq, x, want, wdeq = case(qref.Q6_K, factor, acts, 2000 + factor)
    exact = emu.q6k_single_product(wq, N, K, xq, M, "exact")
    assert normalised_error(exact, want, wdeq, x) < 1e-6
    approx = emu.q6k_single_product(wq, N, K, xq, M, form)
    err = normalised_error(approx, want, wdeq, x)
    assert 1e-6 < err <= TOL_GEMM, err


def test_operand_error_bounds():
    """Per-value bounds of the rounded operands, over every code and scale:
    Q4_K |sc (q - 8) - 4 w8| <= 2; Q6_K |sc (q - 32) - (4096/127) w8| <=
    16 * 4096 / 127 / 256 * 2 + |q - 32| * 8 / 127 (the rounding of w8 and
    of m_j); the 16-bit lanes never overflow."""
    sc = np.arange(64)[:, None]
    q = np.arange(16)[None, :]
    v = sc * (q - 8)
    w8 = np.floor_divide(v + 2, 4)
    assert np.abs(v - 4 * w8).max() <= 2 and w8.min() >= -126 and w8.max() <= 110
    for s in range(-128, 128):
        mj = (127 * s + 8) // 16
        qv = np.arange(64)
        w = (mj * (qv - 32) + 128) // 256
        assert np.abs(mj * (qv - 32)).max() <= 32767
        exact = s * (qv - 32)
        err = np.abs(exact - 4096.0 / 127.0 * w)
        assert (err <= 4096.0 / 127.0 / 2 + np.abs(qv - 32) * 8.0 / 127.0 + 1e-9).all(), s
