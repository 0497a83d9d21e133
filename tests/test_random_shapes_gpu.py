"""Products at seeded random shapes against the CPU oracle, through the C ABI.

Each case draws the type, the weight rows n, the row length k, the activation
rows M, the activation's row stride (contiguous or padded) and whether the
product shares its launch with a second weight, from a fixed seed, so the
kernel choice crosses every line of the dispatch with ragged n and M: the
decode kernels (1-2 rows), the multi-row kernels (to 8), the few-row
matrix-core kernels (Q4_K / Q6_K from 4 rows on weights of 2 MiB, and from
9), the GEMMs (from 33 rows; the 32-value formats from 9) and the
single-pass GEMM (from 129 rows at k >= 2048, cut along K where its tiles
leave CUs idle).

Bounds (normalised by ||w_j||·||x_r||): 1e-3 up to
3 rows, 2e-3 above (the matrix-core products), and each kernel's own: 1e-5
for exact integer sums, 5e-4 with an f16 min term, 2e-3 for the rounded
weight operands. A shared launch gives each weight its own forward's bits.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import TOL_GEMM, TOL_MATVEC, TYPES, normalised_error, weights
from oracle import qref
from swarmllm_amd import GgmlDType, QTensor
from swarmllm_amd._lib import lib

pytestmark = pytest.mark.gpu

DEV = "cuda"
ROWS = [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 13, 16, 17, 24, 31, 32, 33, 40, 64, 100, 128, 129, 160, 257, 300]
N_CASES = 96


def draw_cases():
    rng = np.random.default_rng(20261202)
    names = list(TYPES)
    cases = []
    while len(cases) < N_CASES:
        name = names[int(rng.integers(len(names)))]
        block = 256 if name in ("Q4_K", "Q6_K") else 32
        k = block * int(rng.integers(1, (8192 if block == 256 else 4096) // block + 1))
        rows = ROWS[int(rng.integers(len(ROWS)))]
        n = int(rng.integers(1, 3001))
        # keep the oracle's work to about a second a case
        if n * k > 8_000_000 or rows * n * k > 600_000_000:
            continue
        pad = [0, 0, 4, 1][int(rng.integers(4))]  # floats past each activation row
        shared = bool(rng.integers(2))
        cases.append((name, n, k, rows, pad, shared, int(rng.integers(1 << 30))))
    return cases


CASES = draw_cases()


def bound(kernel: str) -> float:
    """The error a kernel's arithmetic allows (measured on these cases: exact
    sums ~1e-8, the f16 min term ~1e-4, the rounded weight operands 3e-4 to
    6e-4), so a lost or wrong term in an exact kernel fails here rather than
    under the path's looser bound."""
    if "_sp_targets" in kernel or "ONE = true" in kernel:
        return TOL_GEMM  # the single-pass GEMMs and the few-row Q6_K single-product form
    if "launch_gemm_q4k(" in kernel:
        return 5e-4  # the two-pass Q4_K GEMM: its min term's operands in f16
    return 1e-5  # exact integer sums, f32 scaling


def forward_c(qt: QTensor, xs: torch.Tensor, stride: int, k: int, rows: int) -> torch.Tensor:
    """qmm_forward with the activation's row stride, its planned workspace."""
    L = lib()
    n = qt.shape[0]
    out = torch.empty((rows, n), dtype=torch.float32, device=DEV)
    need = ctypes.c_size_t(0)
    t = int(qt.dtype)
    assert L.qmm_forward(t, None, None, stride, None, n, None, 0, ctypes.byref(need), k, n, rows, 0, 0) == 0
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=DEV)
    assert L.qmm_forward(t, qt.data_.data_ptr(), xs.data_ptr(), stride, out.data_ptr(), n, ws.data_ptr(),
                         ws.numel(), ctypes.byref(need), k, n, rows, 1, 0) == 0
    return out


def shared_c(qts, xs: torch.Tensor, stride: int, k: int, rows: int):
    """qmm_forward_shared of the weights over one activation."""
    L = lib()
    cnt = len(qts)
    outs = [torch.empty((rows, q.shape[0]), dtype=torch.float32, device=DEV) for q in qts]
    wp = (ctypes.c_void_p * cnt)(*[q.data_.data_ptr() for q in qts])
    ns = (ctypes.c_int64 * cnt)(*[q.shape[0] for q in qts])
    dp = (ctypes.c_void_p * cnt)(*[o.data_ptr() for o in outs])
    need = ctypes.c_size_t(0)
    t = int(qts[0].dtype)
    assert L.qmm_forward_shared(t, cnt, wp, ns, dp, ns, None, stride, None, 0, ctypes.byref(need), k, rows, 0, 0) == 0
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=DEV)
    assert L.qmm_forward_shared(t, cnt, wp, ns, dp, ns, xs.data_ptr(), stride, ws.data_ptr(), ws.numel(),
                                ctypes.byref(need), k, rows, 1, 0) == 0
    return outs


@pytest.mark.parametrize("name,n,k,rows,pad,shared,seed", CASES,
                         ids=[f"{c[0]}-n{c[1]}-k{c[2]}-m{c[3]}-p{c[4]}{'-sh' if c[5] else ''}" for c in CASES])
def test_random_shape_against_oracle(name, n, k, rows, pad, shared, seed):
    qtype = TYPES[name]
    rng = np.random.default_rng(seed)
    w = weights(rng, n, k)
    wq = qref.from_float(qtype, w)
    qt = QTensor.from_data(wq.tobytes(), (n, k), GgmlDType(qtype), device=DEV)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    stride = k + pad
    xp = np.zeros((rows, stride), np.float32)
    xp[:, :k] = x
    xp[:, k:] = np.float32(1e30)  # never read: a read past the row would show
    xs = torch.from_numpy(xp).to(DEV)
    y = forward_c(qt, xs, stride, k, rows)
    torch.cuda.synchronize()
    want = qref.matmul(qtype, x, wq, n)
    wdeq = qref.to_float(qtype, wq, n * k).reshape(n, k)
    err = normalised_error(y.cpu().numpy(), want, wdeq, x)
    kernel = lib().qmm_last_kernel().decode()
    assert err <= (TOL_MATVEC if rows <= 3 else TOL_GEMM), f"{name} n={n} k={k} rows={rows}: {err} ({kernel})"
    assert err <= bound(kernel), f"{name} n={n} k={k} rows={rows} pad={pad}: {err} ({kernel})"
    if shared:
        n2 = int(rng.integers(1, 700))
        w2 = qref.from_float(qtype, weights(rng, n2, k))
        qt2 = QTensor.from_data(w2.tobytes(), (n2, k), GgmlDType(qtype), device=DEV)
        ya, yb = shared_c([qt, qt2], xs, stride, k, rows)
        yb_own = forward_c(qt2, xs, stride, k, rows)
        torch.cuda.synchronize()
        assert torch.equal(ya, y), "shared launch differs from the weight's own forward"
        assert torch.equal(yb, yb_own), "shared launch differs from the second weight's own forward"
