"""qmm_forward_noalloc (the entry point that allocates nothing: its
activation scratch is the library's static per-GPU array) against
qmm_forward with a caller-owned workspace, through the C ABI.

Bit-identical outputs on two calls in a row, the second with a smaller
input (the array keeps the first call's contents), on products whose
planned workspace is used: the matrix-core GEMMs (Q4_K, 64 rows; Q8_0,
11 rows) and the few-row kernels (Q6_K, 12 rows). A product whose
workspace exceeds the array is rejected with nothing enqueued.
"""
import ctypes

import numpy as np
import pytest
import torch

from swarmllm_amd import GgmlDType, QTensor, fill_normal
from swarmllm_amd._lib import QMM_OK, QMM_WORKSPACE_TOO_SMALL, check, lib

pytestmark = pytest.mark.gpu


def forward_with_workspace(L, t, qt, x, n, k, rows):
    need = ctypes.c_size_t(0)
    check("qmm_forward", L.qmm_forward(t, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, rows, 0, 0))
    ws = torch.empty(max(1, need.value), dtype=torch.uint8, device="cuda")
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


def test_noalloc_rejects_what_exceeds_the_scratch():
    L = lib()
    cap = L.qmm_forward_noalloc_max_bytes()
    assert cap == 16 << 20
    k, n = 32768, 64
    rows = 1024  # a Q8_K activation of 1024 x 32768 needs ~36 MiB
    need = ctypes.c_size_t(0)
    check("qmm_forward", L.qmm_forward(12, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, rows, 0, 0))
    assert need.value > cap
    before = L.qmm_gemm_launches() + L.qmm_matvec_launches()
    # argument checks and the size check happen on the host before anything
    # touches the buffers, so placeholder pointers are never dereferenced
    st = L.qmm_forward_noalloc(12, ctypes.c_void_p(256), ctypes.c_void_p(256), k, ctypes.c_void_p(256), n, k, n,
                               rows, 0)
    assert st == QMM_WORKSPACE_TOO_SMALL
    assert L.qmm_gemm_launches() + L.qmm_matvec_launches() == before
    assert st != QMM_OK
