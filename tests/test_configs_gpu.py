"""BASELINE configs at their full shapes, through the C ABI exactly as
bench.py enqueues them, against the CPU oracle.

- C5 at M = 1: one layer of the Llama-3.3-70B shard (hidden 8192, FFN 28672,
  8 kv heads of 128), its 7 products in bench.py's 4 launches
  (q+k+v and gate+up through qmm_forward_shared, o and down through
  qmm_forward). The launch log proves which decode instantiation served
  each group: the k = 8192 Q4_K rows take the streaming kernel with the next
  row's loads in flight.
- C3's Q6_K down projection (k = 14336) at M = 512 on a 512-row slice of its
  4096 weight rows, activations with 1% outlier channels x20.

Weights are N(0, 0.02) quantized on the device (bit-exact to the oracle's
from_float, tested in test_parity_gpu.py) and read back as GGUF bytes for the
oracle. Tolerance: max |y_gpu - y_cpu| / (||w_j|| ||x_r||), w_j the
dequantized weight row.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import TOL_GEMM, TOL_MATVEC
from oracle import qref
from swarmllm_amd import GgmlDType, QTensor, fill_normal
from swarmllm_amd._lib import check, lib

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14


def quantized(n: int, k: int, t: int, seed: int) -> QTensor:
    w = fill_normal(n * k, seed=seed, std=0.02).reshape(n, k)
    qt = QTensor.quantize(w, GgmlDType(t))
    del w
    return qt


def row_norms(qt: QTensor) -> np.ndarray:
    """||w_j|| of the dequantized rows, computed on the device in f64."""
    return torch.linalg.vector_norm(qt.dequantize().double(), dim=1).cpu().numpy()


def normalised(y: np.ndarray, want: np.ndarray, wn: np.ndarray, x: np.ndarray) -> float:
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    return float(np.max(np.abs(y.astype(np.float64) - want.astype(np.float64)) / (wn[None, :] * xn)))


C5 = {"q": (Q4K, 8192, 8192), "k": (Q4K, 1024, 8192), "v": (Q4K, 1024, 8192), "o": (Q4K, 8192, 8192),
      "gate": (Q4K, 28672, 8192), "up": (Q4K, 28672, 8192), "down": (Q6K, 8192, 28672)}
C5_GROUPS = [(8192, ["q", "k", "v"]), (8192, ["o"]), (8192, ["gate", "up"]), (28672, ["down"])]


@pytest.mark.parametrize("group", range(len(C5_GROUPS)), ids=["qkv", "o", "gate_up", "down"])
def test_c5_decode_layer_m1_full_shapes(group):
    k, names = C5_GROUPS[group]
    L = lib()
    stream = torch.cuda.current_stream().cuda_stream
    ws = {nm: quantized(C5[nm][1], C5[nm][2], C5[nm][0], seed=(5 << 40) | (group << 8) | i)
          for i, nm in enumerate(names)}
    t = C5[names[0]][0]
    x = fill_normal(k, seed=(5 << 40) | (0xA0 + group)).reshape(1, k)
    outs = {nm: torch.empty((1, C5[nm][1]), dtype=torch.float32, device="cuda") for nm in names}
    need = ctypes.c_size_t(0)
    work = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    if len(names) == 1:
        nm = names[0]
        n = C5[nm][1]
        check("qmm_forward", L.qmm_forward(t, ws[nm].data_.data_ptr(), x.data_ptr(), k, outs[nm].data_ptr(), n,
                                           work.data_ptr(), work.numel(), ctypes.byref(need), k, n, 1, 1, stream))
    else:
        cnt = len(names)
        wp = (ctypes.c_void_p * cnt)(*[ws[nm].data_.data_ptr() for nm in names])
        ns = (ctypes.c_int64 * cnt)(*[C5[nm][1] for nm in names])
        dp = (ctypes.c_void_p * cnt)(*[outs[nm].data_ptr() for nm in names])
        check("qmm_forward_shared", L.qmm_forward_shared(t, cnt, wp, ns, dp, ns, x.data_ptr(), k, work.data_ptr(),
                                                         work.numel(), ctypes.byref(need), k, 1, 1, stream))
    kernel = L.qmm_last_kernel().decode()
    torch.cuda.synchronize()
    if t == Q4K:
        # 8192-value rows, more rows than one resident round of waves: the
        # streaming kernel with the next row in flight (PF), two 4096-value
        # halves a lane (T = 2)
        assert "launch_stream_x" in kernel and "PF = true" in kernel and "T = 2" in kernel, kernel
    else:
        assert "mv_q6k" in kernel or "launch_stream" in kernel, kernel
    xh = x.cpu().numpy()
    for nm in names:
        wq = np.frombuffer(ws[nm].data(), np.uint8)
        want = qref.matmul(t, xh, wq, C5[nm][1])
        err = normalised(outs[nm].cpu().numpy(), want, row_norms(ws[nm]), xh)
        assert err <= TOL_MATVEC, f"{nm}: {err}"
        assert err <= 1e-5, f"{nm}: {err}"  # the decode kernels sum the reference's exact integers


def test_c3_q6k_down_projection_m512():
    """C3's down projection (Q6_K, k = 14336) at M = 512: a 512-row slice of
    the 4096 weight rows, the full k and the full 512 activation rows with 1%
    outlier channels x20."""
    from swarmllm_amd import QMatMul

    n, k, rows = 512, 14336, 512
    qt = quantized(n, k, Q6K, seed=(3 << 40) | 6)
    rng = np.random.default_rng(36)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    ch = rng.permutation(k)[: k // 100]
    x[:, ch] *= np.float32(20.0)
    y = QMatMul(qt).forward(torch.from_numpy(x).cuda()).cpu().numpy()
    kernel = lib().qmm_last_kernel().decode()
    assert "launch_gemm_q6k_sp" in kernel, kernel  # the single-pass GEMM (k a multiple of 2048)
    want = qref.matmul(Q6K, x, np.frombuffer(qt.data(), np.uint8), n)
    err = normalised(y, want, row_norms(qt), x)
    assert err <= TOL_GEMM, f"{kernel}: {err}"
    assert err <= 1e-3, f"{kernel}: {err}"  # its one rounding: sc (q - 32) into an int8 operand
