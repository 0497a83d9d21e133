"""The approximate-operand kernels on skewed scales, against the oracle and
against their CPU emulation (tests/sp_emulation.py):
  - the single-pass Q4_K GEMM (w8 = floor((sc (q - 8) + 2) / 4)),
  - the single-pass Q6_K GEMM (w8 = round(m_j (q - 32) / 256)),
  - the few-row Q6_K kernel's single-product form at C5's down k (28672)
    and widths (8, 16 rows),
on weights with one sub-block (Q4_K) or group (Q6_K) per super-block 10 or
100 times the rest, with C3's x20-outlier activations and with activations
concentrated on the small sub-blocks. Each output is held to the GEMM
bound (2e-3 normalised) against the oracle, and to 2e-5 against the
emulation, which pins the kernel to the modelled arithmetic (so the
emulation's margins, measured on the CPU at any size, are the kernel's)."""
import numpy as np
import pytest
import torch

import sp_emulation as emu
from helpers import TOL_GEMM, normalised_error
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor
from swarmllm_amd._lib import lib

pytestmark = pytest.mark.gpu
TO_EMULATION = 2e-5


def run(fmt, n, k, m, factor, acts, seed):
    rng = np.random.default_rng(seed)
    unit = 32 if fmt == qref.Q4_K else 16
    w, big = emu.skewed_weights(rng, n, k, unit, factor)
    x = emu.concentrated_activations(rng, m, k, big, unit) if acts == "small" else emu.outlier_activations(rng, m, k)
    wq = qref.from_float(fmt, w)
    qt = QTensor.from_data(wq.tobytes(), (n, k), GgmlDType(fmt))
    print(f"fmt={fmt} n={n} k={k} m={m} factor={factor} acts={acts}", flush=True)
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    kernel = lib().qmm_last_kernel().decode()
    want = qref.matmul(fmt, x, wq, n)
    wdeq = qref.to_float(fmt, wq, n * k).reshape(n, k)
    xq = qref.quantize_rows(fmt, x)
    return y, kernel, want, wdeq, x, wq, xq


@pytest.mark.parametrize("factor", [10, 100])
@pytest.mark.parametrize("acts", ["outliers", "small"])
def test_q4k_single_pass_gemm_skewed(factor, acts):
    n, k, m = 512, 4096, 256
    y, kernel, want, wdeq, x, wq, xq = run(qref.Q4_K, n, k, m, factor, acts, 3000 + factor)
    assert "launch_gemm_q4k_sp" in kernel, kernel
    assert normalised_error(y, want, wdeq, x) <= TOL_GEMM
    assert normalised_error(y, emu.q4k_single_pass(wq, n, k, xq, m), wdeq, x) <= TO_EMULATION


@pytest.mark.parametrize("factor", [10, 100])
@pytest.mark.parametrize("acts", ["outliers", "small"])
def test_q6k_single_pass_gemm_skewed(factor, acts):
    n, k, m = 512, 4096, 256
    y, kernel, want, wdeq, x, wq, xq = run(qref.Q6_K, n, k, m, factor, acts, 4000 + factor)
    assert "launch_gemm_q6k_sp" in kernel, kernel
    assert normalised_error(y, want, wdeq, x) <= TOL_GEMM
    assert normalised_error(y, emu.q6k_single_product(wq, n, k, xq, m, "gemm"), wdeq, x) <= TO_EMULATION


@pytest.mark.parametrize("rows", [8, 16])
@pytest.mark.parametrize("acts", ["outliers", "small"])
def test_q6k_few_rows_single_product_skewed_at_c5_down_k(rows, acts):
    n, k = 1024, 28672
    y, kernel, want, wdeq, x, wq, xq = run(qref.Q6_K, n, k, rows, 30, acts, 5000 + rows)
    assert "launch_q6" in kernel and "ONE = true" in kernel, kernel
    assert normalised_error(y, want, wdeq, x) <= TOL_GEMM
    assert normalised_error(y, emu.q6k_single_product(wq, n, k, xq, rows, "few_rows"), wdeq, x) <= TO_EMULATION
