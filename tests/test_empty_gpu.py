"""Empty batches through the host API: a product over zero activation rows
returns the empty output of the product's shape ([..., 0, n]) and launches
nothing, for every type and for the shared and GLU forms; a batch with zero
rows between non-empty ones is handled the same. The C ABI itself rejects a
zero-row call (QMM_UNSUPPORTED, checked on the CPU in test_abi_cpu.py), so
the host layer is what must not reach it."""
import numpy as np
import pytest
import torch

from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal, forward_glu
from swarmllm_amd._lib import lib

pytestmark = pytest.mark.gpu

TYPES = [GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.Iq4Nl, GgmlDType.Mxfp4]


def qmm(n, k, t, seed):
    return QMatMul(QTensor.quantize(fill_normal(n * k, seed=seed, std=0.02).reshape(n, k), t))


def launches():
    L = lib()
    return L.qmm_matvec_launches() + L.qmm_gemm_launches()


@pytest.mark.parametrize("t", TYPES, ids=lambda t: t.name)
def test_zero_rows_give_an_empty_output_and_no_launch(t):
    n, k = 96, 512
    mm = qmm(n, k, t, 900 + int(t))
    for shape in [(0, k), (3, 0, k), (0, 2, k)]:
        x = torch.empty(shape, dtype=torch.float32, device="cuda")
        before = launches()
        y = mm.forward(x)
        torch.cuda.synchronize()
        assert tuple(y.shape) == shape[:-1] + (n,) and y.dtype == torch.float32 and y.is_cuda
        assert launches() == before
    # the same weight still computes after the empty calls
    x = fill_normal(2 * k, seed=901).reshape(2, k)
    assert np.isfinite(mm.forward(x).cpu().numpy()).all()


def test_zero_rows_shared_and_glu():
    k = 512
    a, b = qmm(64, k, GgmlDType.Q4K, 910), qmm(32, k, GgmlDType.Q4K, 911)
    x = torch.empty((0, k), dtype=torch.float32, device="cuda")
    before = launches()
    ya, yb = QMatMul.forward_shared(x, [a, b])
    assert tuple(ya.shape) == (0, 64) and tuple(yb.shape) == (0, 32)
    g, u = qmm(64, k, GgmlDType.Q4K, 912), qmm(64, k, GgmlDType.Q4K, 913)
    for act in ("silu", "swiglu_oai", "gelu"):
        assert tuple(forward_glu(x, g, u, act).shape) == (0, 64)
    torch.cuda.synchronize()
    assert launches() == before
