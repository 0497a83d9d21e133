"""qmm_forward_noalloc (the entry point that allocates nothing: its
activation scratch is the library's static per-GPU array) against
qmm_forward with a caller-owned workspace, through the C ABI.

Bit-identical outputs on two calls in a row, the second with a smaller
input (the array keeps the first call's contents), on products whose
planned workspace is used: the matrix-core GEMMs (Q4_K, 64 rows; Q8_0,
11 rows) and the few-row kernels (Q6_K, 12 rows). A single-pass GEMM whose
planned K-split slots do not fit beside the activation (4096 x 4096 at 512
rows: 32 MiB of slots) runs as qmm_forward does with a workspace of the
array's size. A product whose quantized activation exceeds the array is
rejected with nothing enqueued.
"""
import ctypes

import numpy as np
import pytest
import torch

from swarmllm_amd import GgmlDType, QTensor, fill_normal
from swarmllm_amd._lib import QMM_OK, QMM_WORKSPACE_TOO_SMALL, check, lib

pytestmark = pytest.mark.gpu


def forward_with_workspace(L, t, qt, x, n, k, rows, ws_bytes=None):
    """qmm_forward with the workspace it plans, or one of ws_bytes."""
    need = ctypes.c_size_t(0)
    check("qmm_forward", L.qmm_forward(t, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, rows, 0, 0))
    ws = torch.empty(max(1, need.value if ws_bytes is None else ws_bytes), dtype=torch.uint8, device="cuda")
    out = torch.full((rows, n), float("nan"), dtype=torch.float32, device="cuda")
    check("qmm_forward", L.qmm_forward(t, qt.data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n, ws.data_ptr(),
                                       ws.numel(), ctypes.byref(need), k, n, rows, 1,
                                       torch.cuda.current_stream().cuda_stream))
    return out, need.value


def forward_noalloc(L, t, qt, x, n, k, rows):
    out = torch.full((rows, n), float("nan"), dtype=torch.float32, device="cuda")
    check("qmm_forward_noalloc", L.qmm_forward_noalloc(t, qt.data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n, k,
                                                       n, rows, torch.cuda.current_stream().cuda_stream))
    return out


CASES = [  # (type, (n, k, rows) first call, (n, k, rows) second, smaller call)
    (12, (1000, 4096, 64), (300, 2048, 40)),
    (14, (700, 2048, 12), (300, 1024, 9)),
    (8, (500, 1024, 11), (129, 512, 10)),
]


@pytest.mark.parametrize("t,first,second", CASES, ids=["q4k_gemm", "q6k_few_rows", "q8_0_gemm"])
def test_noalloc_equals_forward_on_two_calls(t, first, second):
    L = lib()
    for i, (n, k, rows) in enumerate((first, second)):
        qt = QTensor.quantize(fill_normal(n * k, seed=900 + 10 * t + i, std=0.02).reshape(n, k), GgmlDType(t))
        x = fill_normal(rows * k, seed=950 + 10 * t + i).reshape(rows, k)
        want, need = forward_with_workspace(L, t, qt, x, n, k, rows)
        assert need > 0
        got = forward_noalloc(L, t, qt, x, n, k, rows)
        torch.cuda.synchronize()
        assert not torch.isnan(got).any()
        assert torch.equal(got, want), f"call {i}: {(got - want).abs().max().item()}"


@pytest.mark.parametrize("t", [12, 14], ids=["q4k", "q6k"])
def test_noalloc_gemm_whose_split_slots_do_not_fit(t):
    """4096 x 4096 at 512 rows plans a K split whose slots (32 MiB) do not
    fit the 16 MiB array: the product runs as qmm_forward does with a
    workspace of the array's size (Q4_K uncut, Q6_K on its exact GEMM), bit
    for bit, on two calls in a row."""
    L = lib()
    cap = L.qmm_forward_noalloc_max_bytes()
    n = k = 4096
    rows = 512
    need = ctypes.c_size_t(0)
    check("qmm_forward", L.qmm_forward(t, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, rows, 0, 0))
    assert need.value > cap > L.qmm_act_bytes(L.qmm_act_layout(t, rows), k, rows)
    qt = QTensor.quantize(fill_normal(n * k, seed=970 + t, std=0.02).reshape(n, k), GgmlDType(t))
    x = fill_normal(rows * k, seed=971 + t).reshape(rows, k)
    want, _ = forward_with_workspace(L, t, qt, x, n, k, rows, ws_bytes=cap)
    planned, _ = forward_with_workspace(L, t, qt, x, n, k, rows)
    for call in range(2):
        got = forward_noalloc(L, t, qt, x, n, k, rows)
        torch.cuda.synchronize()
        assert not torch.isnan(got).any()
        assert torch.equal(got, want), f"call {call}: {(got - want).abs().max().item()}"
        if t == 14:
            assert "launch_gemm_q6k(" in L.qmm_last_kernel().decode()
    # against the planned (split) run: the same product summed another way
    scale = float(x.norm(dim=1).max().item()) * float(qt.dequantize().norm(dim=1).max().item())
    assert float((got - planned).abs().max().item()) <= 2e-3 * scale


def test_noalloc_rejects_what_exceeds_the_scratch():
    L = lib()
    cap = L.qmm_forward_noalloc_max_bytes()
    assert cap == 16 << 20
    k, n = 32768, 64
    rows = 1024  # a Q8_K activation of 1024 x 32768 needs ~36 MiB
    need = ctypes.c_size_t(0)
    check("qmm_forward", L.qmm_forward(12, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, rows, 0, 0))
    assert need.value > cap
    w = QTensor.alloc((n, k), GgmlDType.Q4K)
    x = torch.zeros((rows, k), dtype=torch.float32, device="cuda")
    out = torch.full((rows, n), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    before = L.qmm_gemm_launches() + L.qmm_matvec_launches()
    st = L.qmm_forward_noalloc(12, w.data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n, k, n, rows,
                               torch.cuda.current_stream().cuda_stream)
    assert st == QMM_WORKSPACE_TOO_SMALL
    assert L.qmm_gemm_launches() + L.qmm_matvec_launches() == before
    torch.cuda.synchronize()
    assert torch.isnan(out).all()  # nothing was enqueued
    assert st != QMM_OK
