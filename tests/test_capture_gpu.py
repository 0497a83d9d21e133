"""Whole steps of the path captured as one HIP graph (the reference proves a
captured product equals the uncaptured one, src/inference/layers/mod.rs:
8860-8930, under the capture rules of quantized/cuda.rs:841-932).

A decode layer of C2 (7 products in 4 launches at M = 1, with the shared
activations of q/k/v and gate/up), three layers of C5's shapes at M = 8
(the few-row matrix-core kernels), a C3-shaped prefill product at M = 512
(activation quantizer + GEMM inside the graph) and qmm_forward_noalloc at
M = 64 are each captured once and replayed several times. Between replays
the outputs are overwritten with NaN and other products run eagerly, with
synchronisations; every replay must equal the eager result bit for bit.
The eager results are themselves checked against the CPU oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import TOL_GEMM, TOL_MATVEC
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal
from swarmllm_amd._lib import check, lib

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14


def qmat(n, k, t, seed):
    return QMatMul(QTensor.quantize(fill_normal(n * k, seed=seed, std=0.02).reshape(n, k), GgmlDType(t)))


def layer(hidden, ffn, kv, seed):
    return {"q": qmat(hidden, hidden, Q4K, seed), "k": qmat(kv, hidden, Q4K, seed + 1),
            "v": qmat(kv, hidden, Q4K, seed + 2), "o": qmat(hidden, hidden, Q4K, seed + 3),
            "gate": qmat(ffn, hidden, Q4K, seed + 4), "up": qmat(ffn, hidden, Q4K, seed + 5),
            "down": qmat(hidden, ffn, Q6K, seed + 6)}


def step(L, xs):
    """The layer's products in the bench's four launches (q+k+v and gate+up
    share their activation), each output kept for the comparison."""
    x_attn, x_out, x_ffn, x_mid = xs
    q, k, v = QMatMul.forward_shared(x_attn, [L["q"], L["k"], L["v"]])
    o = L["o"].forward(x_out)
    g, u = QMatMul.forward_shared(x_ffn, [L["gate"], L["up"]])
    d = L["down"].forward(x_mid)
    return [q, k, v, o, g, u, d]


def inputs(rows, hidden, ffn, seed):
    return [fill_normal(rows * hidden, seed=seed).reshape(rows, hidden),
            fill_normal(rows * hidden, seed=seed + 1).reshape(rows, hidden),
            fill_normal(rows * hidden, seed=seed + 2).reshape(rows, hidden),
            fill_normal(rows * ffn, seed=seed + 3).reshape(rows, ffn)]


def capture(fn):
    """fn() captured on a side stream (default priority) after a warm-up
    call; returns the graph and the tensors fn returned inside it."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up: workspaces allocated before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = fn()
    torch.cuda.synchronize()
    return g, outs


def replay_and_compare(g, outs, want, disturb, replays=4):
    for r in range(replays):
        for o in outs:
            o.fill_(float("nan"))
        disturb()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), f"replay {r}, output {i}: {(o - w).abs().max().item()}"


def oracle_check(mm, x, y, tol):
    xh = x.cpu().numpy().reshape(-1, x.shape[-1])
    t = int(mm.qtensor.dtype)
    n, k = mm.qtensor.shape
    wq = np.frombuffer(mm.qtensor.data(), np.uint8)
    want = qref.matmul(t, xh, wq, n)
    wn = torch.linalg.vector_norm(mm.qtensor.dequantize().double(), dim=1).cpu().numpy()
    xn = np.linalg.norm(xh.astype(np.float64), axis=1)[:, None]
    err = np.max(np.abs(y.cpu().numpy().reshape(want.shape).astype(np.float64) - want) / (wn[None, :] * xn))
    assert err <= tol, err


def test_capture_c2_decode_layer_m1():
    L = layer(4096, 14336, 1024, seed=7000)
    xs = inputs(1, 4096, 14336, seed=7100)
    want = [t.clone() for t in step(L, xs)]
    other = qmat(300, 1024, Q4K, 7200)
    ox = fill_normal(5 * 1024, seed=7201).reshape(5, 1024)
    g, outs = capture(lambda: step(L, xs))
    replay_and_compare(g, outs, want, lambda: other.forward(ox))
    for name, y, x in (("q", want[0], xs[0]), ("gate", want[4], xs[2]), ("down", want[6], xs[3])):
        oracle_check(L[name], x, y, TOL_MATVEC)


def test_capture_c5_layers_m8():
    layers = [layer(8192, 28672, 1024, seed=7300 + 10 * i) for i in range(3)]
    xs = inputs(8, 8192, 28672, seed=7400)

    def fwd():
        outs = []
        for L in layers:
            outs += step(L, xs)
        return outs

    want = [t.clone() for t in fwd()]
    g, outs = capture(fwd)
    replay_and_compare(g, outs, want, lambda: layers[0]["o"].forward(xs[1][:2]))
    oracle_check(layers[2]["down"], xs[3], want[-1], TOL_MATVEC)


def test_capture_prefill_gemm_m512():
    mm = qmat(2048, 4096, Q4K, 7500)
    x = fill_normal(512 * 4096, seed=7501).reshape(512, 4096)
    want = mm.forward(x).clone()
    assert "gemm_q4k_sp" in lib().qmm_last_kernel().decode()
    g, outs = capture(lambda: [mm.forward(x)])
    replay_and_compare(g, outs, [want], lambda: mm.forward(x[:40]))
    oracle_check(mm, x, want, TOL_GEMM)


def test_capture_noalloc_entry_point():
    """qmm_forward_noalloc exists for callers that cannot allocate, such as
    code under capture: its products replay like qmm_forward's."""
    Lb = lib()
    mm = qmat(1000, 4096, Q4K, 7600)
    x = fill_normal(64 * 4096, seed=7601).reshape(64, 4096)
    n, k = 1000, 4096
    want = mm.forward(x).clone()
    out = torch.empty((64, n), device="cuda")

    def fn():
        check("qmm_forward_noalloc", Lb.qmm_forward_noalloc(Q4K, mm.qtensor.data_.data_ptr(), x.data_ptr(), k,
                                                            out.data_ptr(), n, k, n, 64,
                                                            torch.cuda.current_stream().cuda_stream))
        return [out]

    g, outs = capture(fn)
    replay_and_compare(g, outs, [want], lambda: mm.forward(x[:9]))
