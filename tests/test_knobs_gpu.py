"""The reference's A/B switches of the product dispatch, on the device:
set_force_dmmv (quantized/cuda.rs:29-33: the weight dequantized against the
f32 activation, checked against the oracle's to_float and an f64 product)
and the SWARMLLM_QMATMUL_MMQ switches (cuda.rs:737-872), each setting in a
fresh process (tests/knob_child.py) since the environment is read once.
Where a switch sends a product to the decode kernels, its rows equal the
1-row products bit for bit (the decode kernels do not depend on the batch
width); where it sends one to a matrix-core kernel, the result is checked
against the oracle.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from helpers import TOL_GEMM, normalised_error
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal, forward_glu, set_force_dmmv
from swarmllm_amd._lib import lib

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
TYPES = {"Q8_0": 8, "Q4_K": 12, "Q6_K": 14, "IQ4_NL": 20, "MXFP4": 39}
# f32 sums of k products of exact to_float values against an f64 product
TOL_DMMV = 1e-5


def qmat(t, n, k, seed):
    return QMatMul(QTensor.quantize(fill_normal(n * k, seed=seed, std=0.02).reshape(n, k), GgmlDType(t)))


def dmmv_error(mm, x, y):
    n, k = mm.qtensor.shape
    wd = qref.to_float(int(mm.qtensor.dtype), np.frombuffer(mm.qtensor.data(), np.uint8), n * k).reshape(n, k)
    xh = x.cpu().numpy().reshape(-1, k)
    want = xh.astype(np.float64) @ wd.astype(np.float64).T
    return normalised_error(y.cpu().numpy().reshape(want.shape), want, wd, xh)


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows", [1, 3, 11])
def test_force_dmmv_dequantizes_against_the_f32_activation(name, rows):
    t = TYPES[name]
    n, k = 96, 512
    mm = qmat(t, n, k, 100 + t)
    x = fill_normal(rows * k, seed=200 + rows).reshape(rows, k)
    set_force_dmmv(True)
    try:
        y = mm.forward(x)
        torch.cuda.synchronize()
        assert b"launch_dmmv" in lib().qmm_last_kernel()
    finally:
        set_force_dmmv(False)
    assert dmmv_error(mm, x, y) <= TOL_DMMV
    # the flag is off again: the quantized path, and not the same bits
    y2 = mm.forward(x)
    torch.cuda.synchronize()
    assert b"launch_dmmv" not in lib().qmm_last_kernel()
    assert not torch.equal(y, y2)


def test_force_dmmv_shared_and_glu_forms():
    k = 1024
    gate, up = qmat(12, 64, k, 301), qmat(12, 64, k, 302)
    x = fill_normal(k, seed=303).reshape(1, k)
    set_force_dmmv(True)
    try:
        g1, u1 = gate.forward(x), up.forward(x)
        g2, u2 = QMatMul.forward_shared(x, [gate, up])
        h = forward_glu(x, gate, up, "silu")
        torch.cuda.synchronize()
    finally:
        set_force_dmmv(False)
    assert torch.equal(g1, g2) and torch.equal(u1, u2)
    want = (g1 / (1.0 + torch.exp(-g1))) * u1
    assert torch.allclose(h, want, rtol=1e-6, atol=1e-7)
    assert dmmv_error(gate, x, g1) <= TOL_DMMV


def run_child(env, specs, tmp_path):
    full = {k: v for k, v in os.environ.items() if not k.startswith("SWARMLLM_QMATMUL_MMQ")}
    full.update(env)
    full["PYTHONPATH"] = ROOT + (os.pathsep + full["PYTHONPATH"] if full.get("PYTHONPATH") else "")
    out = str(tmp_path / "child.npz")
    print(f"child with {env}", flush=True)
    res = subprocess.run([sys.executable, "-u", os.path.join(HERE, "knob_child.py"), json.dumps(specs), out],
                         env=full, cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    z = np.load(out)
    return [(z[f"y{i}"], tuple(int(v) for v in z[f"launches{i}"])) for i in range(len(specs))]


def same_inputs(spec):
    n, k, rows = spec["n"], spec["k"], spec["rows"]
    mm = qmat(spec["type"], n, k, spec["seed"])
    x = fill_normal(rows * k, seed=spec["seed"] + 1).reshape(rows, k)
    return mm, x


def per_row(mm, x):
    return np.concatenate([mm.forward(x[r:r + 1]).cpu().numpy() for r in range(x.shape[0])])


def oracle_error(mm, x, y):
    n, k = mm.qtensor.shape
    t = int(mm.qtensor.dtype)
    wq = np.frombuffer(mm.qtensor.data(), np.uint8)
    xh = x.cpu().numpy()
    want = qref.matmul(t, xh, wq, n)
    wd = qref.to_float(t, wq, n * k).reshape(n, k)
    return normalised_error(y, want, wd, xh)


def test_mmq_off_and_max_rows_keep_products_on_the_decode_kernels(tmp_path):
    specs = [{"type": 12, "n": 512, "k": 1024, "rows": 40, "seed": 11},
             {"type": 8, "n": 256, "k": 512, "rows": 20, "seed": 12}]
    for (y, (mv, gm)), spec in zip(run_child({"SWARMLLM_QMATMUL_MMQ": "off"}, specs, tmp_path), specs):
        assert gm == 0 and mv == (spec["rows"] + 7) // 8
        mm, x = same_inputs(spec)
        assert np.array_equal(y.view(np.uint32), per_row(mm, x).view(np.uint32))
    specs = [{"type": 12, "n": 512, "k": 1024, "rows": 40, "seed": 13},
             {"type": 12, "n": 512, "k": 1024, "rows": 16, "seed": 14}]
    got = run_child({"SWARMLLM_QMATMUL_MMQ_MAX_ROWS": "16"}, specs, tmp_path)
    (y40, (mv40, gm40)), (y16, (mv16, gm16)) = got
    assert gm40 == 0 and mv40 == 5
    mm, x = same_inputs(specs[0])
    assert np.array_equal(y40.view(np.uint32), per_row(mm, x).view(np.uint32))
    # 16 rows: the few-row matrix-core kernel, as without the switch
    assert gm16 == 1 and mv16 == 0
    mm, x = same_inputs(specs[1])
    assert np.array_equal(y16.view(np.uint32), mm.forward(x).cpu().numpy().view(np.uint32))


def test_mmq_min_rows_and_bytes_move_the_few_rows_line(tmp_path):
    specs = [{"type": 12, "n": 256, "k": 1024, "rows": 2, "seed": 21},
             {"type": 14, "n": 256, "k": 1024, "rows": 3, "seed": 22},
             {"type": 8, "n": 256, "k": 512, "rows": 5, "seed": 23},
             {"type": 39, "n": 128, "k": 512, "rows": 7, "seed": 24}]
    got = run_child({"SWARMLLM_QMATMUL_MMQ_MIN_ROWS": "2", "SWARMLLM_QMATMUL_MMQ_FEW_ROWS_BYTES": "0"}, specs,
                    tmp_path)
    for (y, (mv, gm)), spec in zip(got, specs):
        assert (mv, gm) == (0, 1), spec
        mm, x = same_inputs(spec)
        assert oracle_error(mm, x, y) <= TOL_GEMM, spec
    # without the switches the same products stay on the decode kernels
    for spec in specs:
        mm, x = same_inputs(spec)
        gm0 = lib().qmm_gemm_launches()
        mm.forward(x)
        assert lib().qmm_gemm_launches() == gm0, spec


def test_mmq_captured_off_keeps_captured_few_rows_products_on_the_decode_kernels(tmp_path):
    # a 2.36 MB Q4_K weight at 6 rows: past the default few-rows line
    spec = {"type": 12, "n": 4096, "k": 1024, "rows": 6, "seed": 31}
    got = run_child({"SWARMLLM_QMATMUL_MMQ_CAPTURED": "0"}, [spec, dict(spec, capture=True)], tmp_path)
    (ye, (mve, gme)), (yc, (mvc, gmc)) = got
    assert (mve, gme) == (0, 1)  # eager: the few-row matrix-core kernel
    assert (mvc, gmc) == (1, 0)  # captured: the decode kernel
    mm, x = same_inputs(spec)
    assert np.array_equal(yc.view(np.uint32), per_row(mm, x).view(np.uint32))
    assert np.array_equal(ye.view(np.uint32), mm.forward(x).cpu().numpy().view(np.uint32))
    assert oracle_error(mm, x, ye) <= TOL_GEMM


def test_exact_forms_switch(tmp_path):
    """SWARMLLM_QMATMUL_EXACT=1: the products the approximate-operand kernels
    take by default (the single-pass Q4_K / Q6_K GEMMs from 129 rows, the
    few-row Q6_K single-product form from k = 2048) run on the exact
    kernels, within the exact kernels' bound of the oracle."""
    specs = [{"type": 12, "n": 1024, "k": 4096, "rows": 256, "seed": 41},
             {"type": 14, "n": 1024, "k": 4096, "rows": 256, "seed": 42},
             {"type": 14, "n": 2048, "k": 4096, "rows": 8, "seed": 43}]
    got = run_child({"SWARMLLM_QMATMUL_EXACT": "1"}, specs, tmp_path)
    kernels = np.load(str(tmp_path / "child.npz"))
    names = [str(kernels[f"kernel{i}"]) for i in range(len(specs))]
    assert "launch_gemm_q4k(" in names[0], names[0]
    assert "launch_gemm_q6k(" in names[1], names[1]
    assert "launch_q6" in names[2] and "ONE = false" in names[2], names[2]
    for (y, _), spec in zip(got, specs):
        mm, x = same_inputs(spec)
        assert oracle_error(mm, x, y) <= 5e-4, spec
    # without the switch (this process) the same products take the
    # approximate forms
    assert lib().qmm_exact_forms() == 0
    for spec, want in zip(specs, ("launch_gemm_q4k_sp", "launch_gemm_q6k_sp", "ONE = true")):
        mm, x = same_inputs(spec)
        mm.forward(x)
        assert want in lib().qmm_last_kernel().decode(), spec
