"""The gated activation act(gate) * up on the device, through the C ABI.

- qmm_glu (the elementwise kernel) against the CPU oracle (oracle/qref_glu.c,
  pinned in test_glu_oracle.py) within the reference's own bound for a
  card's result, |gpu - cpu| <= 1e-5 max(|cpu|, 1) (fast_math.rs:612-620: a
  card's exp is not the host's), NaN where the oracle has NaN;
- qmm_forward_glu, the gate+up+GLU launch, equal bit for bit to the gate and
  up products of qmm_forward_shared followed by qmm_glu: fused for Q4_K at
  1-2 rows (C2's and C5's gate/up shapes), and the two-launch form
  otherwise (more rows, other types, an unaligned activation);
- and end to end against the oracle's products and activation.
"""
import numpy as np
import pytest
import torch

from helpers import weights
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal, forward_glu, glu
from swarmllm_amd._lib import lib

pytestmark = pytest.mark.gpu

ACTS = ["silu", "swiglu_oai", "gelu"]


def card_bound(got: np.ndarray, want: np.ndarray) -> None:
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    inf = np.isinf(want)
    assert np.array_equal(got[inf], want[inf])  # infinite where the oracle is, with its sign
    fin = ~(nan | inf)
    g, w = got[fin].astype(np.float64), want[fin].astype(np.float64)
    assert np.all(np.abs(g - w) <= 1e-5 * np.maximum(np.abs(w), 1.0)), np.max(np.abs(g - w))


@pytest.mark.parametrize("act", ACTS)
def test_glu_elementwise_matches_oracle(act):
    from test_glu_oracle import swiglu_inputs

    rng = np.random.default_rng(3)
    g0, u0 = swiglu_inputs()
    g1 = (rng.standard_normal(2880 * 8) * 6).astype(np.float32)  # the reference's card test: sigma 6
    u1 = (rng.standard_normal(2880 * 8) * 6).astype(np.float32)
    edge = np.array([0.0, -0.0, 100.0, -100.0, np.nan, 1.0, np.inf, -np.inf, 1e-30], np.float32)
    g = np.concatenate([g0, g1, edge, np.ones_like(edge)])
    u = np.concatenate([u0, u1, np.ones_like(edge), edge])
    out = glu(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda(), act).cpu().numpy()
    card_bound(out, qref.glu(act, g, u))


def glu_pair(n, k, t, seed):
    wg = fill_normal(n * k, seed=seed, std=0.02).reshape(n, k)
    wu = fill_normal(n * k, seed=seed + 1, std=0.02).reshape(n, k)
    return QMatMul(QTensor.quantize(wg, GgmlDType(t))), QMatMul(QTensor.quantize(wu, GgmlDType(t)))


def composed(x, gate, up, act):
    g, u = QMatMul.forward_shared(x, [gate, up])
    return glu(g.contiguous(), u.contiguous(), act)


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("n,k,rows", [(14336, 4096, 1), (14336, 4096, 2), (28672, 8192, 1), (300, 256, 2),
                                      (5000, 2048, 1)])
def test_fused_gate_up_glu_equals_composition(act, n, k, rows):
    gate, up = glu_pair(n, k, 12, seed=(k << 8) | rows)
    x = fill_normal(rows * k, seed=rows + 17).reshape(rows, k)
    y = forward_glu(x, gate, up, act)
    assert "launch_glu_x" in lib().qmm_last_kernel().decode()  # one launch
    assert torch.equal(y, composed(x, gate, up, act))


@pytest.mark.parametrize("t,k,rows", [(12, 4096, 5), (12, 16384, 1), (14, 1024, 1), (14, 1024, 40), (8, 2880, 1),
                                      (39, 2880, 12), (20, 512, 3)])
def test_two_launch_gate_up_glu_equals_composition(t, k, rows):
    gate, up = glu_pair(700, k, t, seed=t * 100 + rows)
    x = fill_normal(rows * k, seed=rows + 5).reshape(rows, k)
    for act in ACTS:
        y = forward_glu(x, gate, up, act)
        assert "launch_glu(" in lib().qmm_last_kernel().decode()
        assert torch.equal(y, composed(x, gate, up, act))


def test_unaligned_activation_takes_the_two_launch_form():
    gate, up = glu_pair(500, 1024, 12, seed=9)
    buf = fill_normal(2 * 1024 + 1, seed=3)
    x = buf[1:1025].reshape(1, 1024)  # 4 bytes past an aligned start
    y = forward_glu(x, gate, up, "silu")
    assert "launch_glu(" in lib().qmm_last_kernel().decode()
    assert torch.equal(y, composed(x, gate, up, "silu"))


@pytest.mark.parametrize("act", ACTS)
def test_fused_gate_up_glu_against_oracle(act):
    """End to end: the oracle's gate and up products (the reference's
    integers) and its activation. The products agree within ~1e-6 of
    ||w|| ||x|| (the decode kernels); through act that bounds the gap by
    tol * (|act'(g)| |u| ||w_g|| ||x|| + |act(g)| ||w_u|| ||x||)."""
    n, k = 2048, 4096
    rng = np.random.default_rng(11)
    wg, wu = weights(rng, n, k), weights(rng, n, k)
    qg, qu = qref.from_float(qref.Q4_K, wg), qref.from_float(qref.Q4_K, wu)
    gate = QMatMul(QTensor.from_data(qg.tobytes(), (n, k), GgmlDType.Q4K, device="cuda"))
    up = QMatMul(QTensor.from_data(qu.tobytes(), (n, k), GgmlDType.Q4K, device="cuda"))
    x = rng.standard_normal((1, k)).astype(np.float32)
    y = forward_glu(torch.from_numpy(x).cuda(), gate, up, act).cpu().numpy().astype(np.float64)
    G, U = qref.matmul(qref.Q4_K, x, qg, n), qref.matmul(qref.Q4_K, x, qu, n)
    want = qref.glu(act, G.astype(np.float32), U.astype(np.float32)).astype(np.float64)
    ng = np.linalg.norm(qref.to_float(qref.Q4_K, qg, n * k).reshape(n, k).astype(np.float64), axis=1)
    nu = np.linalg.norm(qref.to_float(qref.Q4_K, qu, n * k).reshape(n, k).astype(np.float64), axis=1)
    nx = np.linalg.norm(x.astype(np.float64))
    gd, ud = G.astype(np.float64), U.astype(np.float64)
    slope = 1.1 + 0.25 * np.abs(gd)  # bounds |act'(g)| for all three on these magnitudes
    scale = slope * (np.abs(ud) + 1.0) * ng * nx + (np.abs(gd) + 1.0) * (np.abs(ud) + 1.0) * nu * nx
    assert np.all(np.abs(y - want) <= 1e-5 * scale + 1e-6 * np.abs(want)), np.max(np.abs(y - want) / scale)
