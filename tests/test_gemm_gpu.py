"""The prefill GEMMs (int8 matrix cores) against the CPU oracle, through the
C ABI: qmm_forward runs them for Q4_K weights from 33 rows (the two-pass
kernel to 128 rows, the single-pass kernel from 129 rows at k >= 2048) and
for Q6_K weights from 33 rows; the few-row kernels below 33.

Tolerance (for the MFMA GEMM): max
|y_gpu - y_cpu| / (||w_j|| * ||x_r||) <= 2e-3. The GEMM multiplies the same
integers as the reference (Q8_K activation, exact int32 super-block sums);
its one approximation is the min term, whose operands dy*S_j and
-dmin*m_j enter its f16 MFMA rounded to f16 (2^-11 relative). An emulation
of exactly that arithmetic in numpy lands within 1e-9 of the GPU on these
cases (5e-8 against the oracle with the min term exact, 1.4e-4 with it in
f16), so the tests also assert a bound of 5e-4 that a lost or wrong term
would break.
"""
import zlib

import numpy as np
import pytest
import torch

from helpers import TOL_GEMM, normalised_error, weights
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor
from swarmllm_amd._lib import lib

pytestmark = pytest.mark.gpu

DEV = "cuda"
TIGHT = 5e-4  # the f16 rounding of the min term's operands, with room


def upload(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def q4k(w: np.ndarray):
    wq = qref.from_float(qref.Q4_K, w)
    return QTensor.from_data(wq.tobytes(), w.shape, GgmlDType.Q4K, device=DEV), wq


def activations(rng, rows: int, k: int, outliers: bool = False) -> np.ndarray:
    x = rng.standard_normal((rows, k)).astype(np.float32)
    if outliers:  # BASELINE C3: 1% of channels scaled x20 in every row
        ch = rng.permutation(k)[: max(1, k // 100)]
        x[:, ch] *= np.float32(20.0)
    return x


GEMM_SHAPES = [  # (k, n, rows): tails in M and N, one and many super-blocks
    (256, 128, 9), (256, 7, 9), (1024, 200, 16), (4096, 300, 33), (2560, 96, 64),
    (4096, 1000, 130), (14336, 136, 40), (512, 384, 257),
]


@pytest.mark.parametrize("k,n,rows", GEMM_SHAPES)
def test_q4k_gemm_parity(k, n, rows):
    rng = np.random.default_rng(zlib.crc32(f"gemm-{k}-{n}-{rows}".encode()))
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = q4k(w)
    L = lib()
    before = L.qmm_gemm_launches()
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert L.qmm_gemm_launches() == before + 1, "the MFMA GEMM did not run"
    want = qref.matmul(qref.Q4_K, x, wq, n)
    wdeq = qref.to_float(qref.Q4_K, wq, n * k).reshape(n, k)
    err = normalised_error(y, want, wdeq, x)
    assert err <= TOL_GEMM, f"k={k} n={n} rows={rows}: {err}"
    # from 129 rows and k >= 2048 the single-pass kernel runs (its bound below)
    assert err <= (TIGHT_SP if rows >= 129 and k >= 2048 else TIGHT), f"k={k} n={n} rows={rows}: {err}"


#: the single-pass GEMM (from 129 rows) rounds sc*(q-8) to a multiple of 4
#: before its one int8 pass; a numpy emulation of that arithmetic on C3-like
#: inputs (outlier channels x20) gives a normalised error of at most 4.2e-4
#: (k = 4096) and 2.4e-4 (k = 14336). Half the 2e-3 budget holds it with room,
#: and a wrong sub-block scale, nibble or offset lands far above it.
TIGHT_SP = 1e-3

SP_SHAPES = [  # (k, n, rows): one and two row tiles, row and weight-row tails, the XCD remap (tiles % 8 == 0)
    (4096, 300, 129), (2048, 7, 200), (2560, 1000, 300), (14336, 136, 256), (4096, 2048, 512), (3072, 4100, 383),
]


@pytest.mark.parametrize("k,n,rows", SP_SHAPES)
def test_q4k_single_pass_gemm_parity(k, n, rows):
    rng = np.random.default_rng(zlib.crc32(f"gemm-sp-{k}-{n}-{rows}".encode()))
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = q4k(w)
    L = lib()
    before = L.qmm_gemm_launches()
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert L.qmm_gemm_launches() == before + 1, "the MFMA GEMM did not run"
    assert "gemm_q4k_sp" in L.qmm_last_kernel().decode()
    want = qref.matmul(qref.Q4_K, x, wq, n)
    wdeq = qref.to_float(qref.Q4_K, wq, n * k).reshape(n, k)
    err = normalised_error(y, want, wdeq, x)
    assert err <= TOL_GEMM, f"k={k} n={n} rows={rows}: {err}"
    assert err <= TIGHT_SP, f"k={k} n={n} rows={rows}: {err}"


def test_q4k_single_pass_gemm_row_scales_of_any_size():
    """Rows scaled by 1e-30, 1e-6, 1e3 and 1e30 (each row's f16 operands are
    brought into range by a power of two of its own), and an all-zero row."""
    k, n, rows = 2048, 256, 160
    rng = np.random.default_rng(91)
    qt, wq = q4k(weights(rng, n, k))
    x = rng.standard_normal((rows, k)).astype(np.float32)
    for r, s in ((0, 1e-30), (1, 1e-6), (2, 1e3), (3, 1e30)):
        x[r] *= np.float32(s)
    x[4] = 0.0
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert "gemm_q4k_sp" in lib().qmm_last_kernel().decode()
    assert np.all(y[4] == 0.0)
    want = qref.matmul(qref.Q4_K, x, wq, n)
    wdeq = qref.to_float(qref.Q4_K, wq, n * k).reshape(n, k)
    keep = [r for r in range(rows) if r != 4]
    err = normalised_error(y[keep], want[keep], wdeq, x[keep])
    assert err <= TIGHT_SP, err


def test_q4k_gemm_c3_gate_full_size():
    """BASELINE C3's gate projection: Q4_K 14336 x 4096 at M = 512, activations
    with 1% outlier channels x20; the weight quantized on the device."""
    from swarmllm_amd import fill_normal

    n, k, rows = 14336, 4096, 512
    w = fill_normal(n * k, seed=3 << 40, std=0.02).reshape(n, k)
    qt = QTensor.quantize(w, GgmlDType.Q4K)
    del w
    rng = np.random.default_rng(3)
    x = activations(rng, rows, k, outliers=True)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    wq = np.frombuffer(qt.data(), np.uint8)
    want = qref.matmul(qref.Q4_K, x, wq, n)
    wdeq = qt.dequantize().cpu().numpy()
    err = normalised_error(y, want, wdeq, x)
    assert err <= TOL_GEMM
    assert "gemm_q4k_sp" in lib().qmm_last_kernel().decode()
    assert err <= TIGHT_SP, err


def test_q4k_gemm_rows_are_independent_and_close_to_the_decode_kernel():
    """Within one GEMM call a row's result does not depend on its place in the
    batch (the reference's qmm_batch: identical rows, identical outputs), and
    across the switch from the decode kernel (<= 8 rows) to the GEMM the
    results differ by the GEMM's f16 min term only (the reference allows a
    deviation at its own kernel switch, quantized_tests.rs:244-251)."""
    k, n = 4096, 300
    rng = np.random.default_rng(12)
    qt, _ = q4k(weights(rng, n, k))
    mm = QMatMul(qt)
    x6 = rng.standard_normal((6, k)).astype(np.float32)
    x12 = upload(np.concatenate([x6, x6]))
    y12 = mm.forward(x12)
    assert torch.equal(y12[:6], y12[6:])
    y6 = mm.forward(upload(x6))
    wdeq = qt.dequantize().cpu().numpy()
    assert normalised_error(y12[:6].cpu().numpy(), y6.cpu().numpy(), wdeq, x6) <= TIGHT


def test_q4k_gemm_through_forward_shared():
    k = 1024
    rng = np.random.default_rng(13)
    mats = [QMatMul(q4k(weights(rng, n, k))[0]) for n in (64, 200, 33)]
    x = upload(rng.standard_normal((20, k)).astype(np.float32))
    shared = QMatMul.forward_shared(x, mats)
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))


def plan_bytes(qt, k, n, rows):
    import ctypes

    need = ctypes.c_size_t(0)
    assert lib().qmm_forward(qref.Q4_K, None, None, k, None, n, None, 0, ctypes.byref(need), k, n, rows, 0, 0) == 0
    return need.value


# (n, rows, k): cut in 4 (k = 4096), and in 2 (k = 2048 and 6144: parts of at
# least 4 super-blocks, a whole number of pairs each)
@pytest.mark.parametrize("n,rows,k", [(1024, 512, 4096), (4096, 512, 4096), (200, 300, 4096), (1024, 512, 2048),
                                      (512, 300, 6144)])
def test_q4k_gemm_cut_along_k(n, rows, k):
    """Products whose tiles fill at most half the CUs (q/k/v/o of a prefill)
    are cut along K when the workspace holds the split slots (forward plans
    them): each part writes its partial tile to a slot and a second launch
    adds the slots in part order. Against the oracle; bit-identical run to
    run; within 1e-5 of the uncut product from the same quantized
    activation (qmm_matmul: the same integers and f32 steps, only the order
    of the partial sums differs)."""
    from swarmllm_amd import _lib
    from swarmllm_amd.qtensor import quantize_act

    rng = np.random.default_rng(zlib.crc32(f"gemm-split-{n}-{rows}-{k}".encode()))
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = q4k(w)
    L = lib()
    assert plan_bytes(qt, k, n, rows) > L.qmm_act_bytes(_lib.ACT_Q8K, k, rows), "no split slots planned"
    mm = QMatMul(qt)
    xt = upload(x)
    y1 = mm.forward(xt).clone()
    assert "gemm_q4k_sp" in L.qmm_last_kernel().decode()
    y2 = mm.forward(xt)
    assert torch.equal(y1, y2)
    xq = quantize_act(xt, _lib.ACT_Q8K)
    uncut = torch.empty((rows, n), dtype=torch.float32, device=DEV)
    assert L.qmm_matmul(qref.Q4_K, qt.data_.data_ptr(), xq.data_ptr(), uncut.data_ptr(), n, k, n, rows,
                        torch.cuda.current_stream().cuda_stream) == 0
    wdeq = qref.to_float(qref.Q4_K, wq, n * k).reshape(n, k)
    y = y1.cpu().numpy()
    assert normalised_error(y, uncut.cpu().numpy(), wdeq, x) <= 1e-5
    want = qref.matmul(qref.Q4_K, x, wq, n)
    err = normalised_error(y, want, wdeq, x)
    assert err <= TOL_GEMM
    assert err <= TIGHT_SP, err


@pytest.mark.parametrize("ns", [(4096, 1024, 1024), (4096, 4096), (4096, 4096, 4096, 4096), (2048, 2048),
                                (14336, 14336)])
def test_q4k_gemm_cut_along_k_shared_equals_forward(ns):
    """Weights sharing one launch at M = 512 give each weight's own forward
    bits: a weight's K split does not depend on the weights sharing its
    launch, nor on how many of a tile's splits one workgroup computes (q+k+v
    and the 4096-row pairs and quadruples have more split workgroups than
    CUs, so workgroups there take 2 or 4 consecutive splits; gate+up's 448
    unsplit tiles run as they do alone)."""
    k, rows = 4096, 512
    rng = np.random.default_rng(15)
    mats = [QMatMul(q4k(weights(rng, n, k))[0]) for n in ns]
    x = upload(activations(rng, rows, k, outliers=True))
    before = lib().qmm_gemm_launches()
    shared = QMatMul.forward_shared(x, mats)
    assert lib().qmm_gemm_launches() == before + 1, "q/k/v did not share one launch"
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))


def test_q4k_gemm_uncut_with_only_the_activation_workspace():
    """qmm_forward_noalloc's 16 MiB scratch holds the activation of an
    o-shaped product at M = 512 but not its split slots: the product runs
    uncut, with qmm_matmul's bits."""
    from swarmllm_amd import _lib
    from swarmllm_amd.qtensor import quantize_act

    n, k, rows = 4096, 4096, 512
    rng = np.random.default_rng(16)
    qt, _ = q4k(weights(rng, n, k))
    L = lib()
    assert plan_bytes(qt, k, n, rows) > L.qmm_forward_noalloc_max_bytes()
    x = upload(activations(rng, rows, k))
    st = torch.cuda.current_stream().cuda_stream
    out = torch.empty((rows, n), dtype=torch.float32, device=DEV)
    assert L.qmm_forward_noalloc(qref.Q4_K, qt.data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n, k, n, rows,
                                 st) == 0
    xq = quantize_act(x, _lib.ACT_Q8K)
    uncut = torch.empty((rows, n), dtype=torch.float32, device=DEV)
    assert L.qmm_matmul(qref.Q4_K, qt.data_.data_ptr(), xq.data_ptr(), uncut.data_ptr(), n, k, n, rows, st) == 0
    assert torch.equal(out, uncut)


@pytest.mark.parametrize("rows", [1, 2, 5, 8, 9, 40])
def test_matmul_from_a_quantized_activation_equals_forward(rows):
    """qmm_matmul (the product from qmm_quantize_act's planes, the
    swarm_mmq_quantize + swarm_mmq_matmul pair) gives forward's bits."""
    from swarmllm_amd import _lib
    from swarmllm_amd.qtensor import quantize_act

    k, n = 1024, 200
    rng = np.random.default_rng(14 + rows)
    qt, _ = q4k(weights(rng, n, k))
    x = upload(rng.standard_normal((rows, k)).astype(np.float32))
    xq = quantize_act(x, _lib.ACT_Q8K)
    out = torch.empty((rows, n), dtype=torch.float32, device=DEV)
    st = lib().qmm_matmul(qref.Q4_K, qt.data_.data_ptr(), xq.data_ptr(), out.data_ptr(), n, k, n, rows,
                          torch.cuda.current_stream().cuda_stream)
    assert st == 0
    assert torch.equal(out, QMatMul(qt).forward(x))


# ---------------------------------------------------------------------------
# the skinny matrix-core kernel: 4-8 rows on weights of 2 MiB or more (the
# reference's few-rows line, quantized/cuda.rs:775-839) and 9-32 rows
# ---------------------------------------------------------------------------
SKINNY_SHAPES = [  # (k, n, rows): past the 2 MiB line at 4-8 rows; ragged n; one and two 16-row tiles
    (4096, 2048, 4), (4096, 2050, 5), (8192, 1030, 8), (2048, 4100, 7), (256, 100, 9), (4096, 300, 16),
    (14336, 64, 17), (1024, 500, 24), (8192, 129, 32),
]


@pytest.mark.parametrize("k,n,rows", SKINNY_SHAPES)
def test_q4k_skinny_parity(k, n, rows):
    rng = np.random.default_rng(zlib.crc32(f"skinny-{k}-{n}-{rows}".encode()))
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = q4k(w)
    L = lib()
    before = L.qmm_gemm_launches()
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert L.qmm_gemm_launches() == before + 1, "the matrix-core kernel did not run"
    want = qref.matmul(qref.Q4_K, x, wq, n)
    wdeq = qref.to_float(qref.Q4_K, wq, n * k).reshape(n, k)
    err = normalised_error(y, want, wdeq, x)
    assert err <= TIGHT, f"k={k} n={n} rows={rows}: {err}"


def test_q4k_small_weight_few_rows_stay_on_the_decode_kernels():
    """Below 2 MiB, 4-8 rows keep the decode kernels (batch-invariant)."""
    rng = np.random.default_rng(5)
    qt, _ = q4k(weights(rng, 256, 4096))  # 576 KiB
    L = lib()
    before = L.qmm_gemm_launches()
    QMatMul(qt).forward(upload(activations(rng, 8, 4096)))
    assert L.qmm_gemm_launches() == before


@pytest.mark.parametrize("rows", [4, 8, 13, 16])
def test_q4k_skinny_c5_gate_projection(rows):
    """BASELINE C5's gate projection (28672 x 8192 Q4_K, a wide weight: the
    copy-staged kernel) at the speculative-verification widths and at the
    few-rows line's 4 rows and a ragged 13."""
    rng = np.random.default_rng(50 + rows)
    w = weights(rng, 28672, 8192)
    x = activations(rng, rows, 8192)
    qt, wq = q4k(w)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert "launch_sk_dma" in lib().qmm_last_kernel().decode()  # the copy-staged kernel
    want = qref.matmul(qref.Q4_K, x, wq, 28672)
    wdeq = qref.to_float(qref.Q4_K, wq, 28672 * 8192).reshape(28672, 8192)
    assert normalised_error(y, want, wdeq, x) <= TIGHT


@pytest.mark.parametrize("rows", [4, 8, 13, 16])
def test_q4k_skinny_narrow_c5_products(rows):
    """BASELINE C5's narrow Q4_K products (q 8192 x 8192, k and v 1024 x 8192
    through one shared launch, o 8192 x 8192) at the few-row widths: the
    narrow-weight kernel that copies each wave's operands to LDS, against the
    oracle, and shared equal to each weight's own forward."""
    from swarmllm_amd import fill_normal

    k = 8192
    mats, wqs = [], []
    for n in (8192, 1024, 1024):
        qt = QTensor.quantize(fill_normal(n * k, seed=600 + n, std=0.02).reshape(n, k), GgmlDType.Q4K)
        mats.append(QMatMul(qt))
        wqs.append(qt.data_.cpu().numpy())
    rng = np.random.default_rng(610 + rows)
    x = activations(rng, rows, k, outliers=True)
    xs = upload(x)
    shared = QMatMul.forward_shared(xs, mats)
    assert "launch_sk_ks" in lib().qmm_last_kernel().decode()
    for m, wq, y in zip(mats, wqs, shared):
        n = y.shape[-1]
        assert torch.equal(y, m.forward(xs))
        assert "launch_sk_ks" in lib().qmm_last_kernel().decode()
        want = qref.matmul(qref.Q4_K, x, wq, n)
        wdeq = qref.to_float(qref.Q4_K, wq, n * k).reshape(n, k)
        assert normalised_error(y.cpu().numpy(), want, wdeq, x) <= TIGHT


@pytest.mark.parametrize("rows", [4, 13])
def test_q4k_skinny_copy_staged_ragged_weight(rows):
    """A wide weight (at least 64 rows a CU: the copy-staged kernel) whose
    rows are not a multiple of 16 and whose 16-row tiles are not a multiple
    of the 4 a workgroup takes (16390 rows: 1025 tiles), so the last tile
    is ragged and the last workgroup has dead tiles; against the oracle, and
    shared with a narrow weight equal to each weight's own forward."""
    from swarmllm_amd import fill_normal

    n, k = 16390, 2048
    rng = np.random.default_rng(80 + rows)
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = q4k(w)
    mm = QMatMul(qt)
    y = mm.forward(upload(x))
    assert "launch_sk_dma" in lib().qmm_last_kernel().decode()
    want = qref.matmul(qref.Q4_K, x, wq, n)
    wdeq = qref.to_float(qref.Q4_K, wq, n * k).reshape(n, k)
    assert normalised_error(y.cpu().numpy(), want, wdeq, x) <= TIGHT
    narrow = QMatMul(QTensor.quantize(fill_normal(300 * k, seed=81, std=0.02).reshape(300, k), GgmlDType.Q4K))
    xs = upload(x)
    shared = QMatMul.forward_shared(xs, [mm, narrow])
    assert torch.equal(shared[0], y) and torch.equal(shared[1], narrow.forward(xs))


@pytest.mark.parametrize("rows", [6, 16, 30])
def test_q4k_skinny_shared_activation_equals_forward(rows):
    """q/k/v-like weights through one qmm_forward_shared (grouped skinny
    launches, more weights than one launch takes) equal each weight's own
    forward bit for bit."""
    rng = np.random.default_rng(70 + rows)
    k = 4096
    mats = [QMatMul(q4k(weights(rng, n, k))[0]) for n in (2048, 512, 512, 1040, 2048)]
    x = upload(activations(rng, rows, k))
    shared = QMatMul.forward_shared(x, mats)
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))


@pytest.mark.parametrize("rows", [4, 8, 16])
def test_q4k_skinny_wide_weights_shared_equals_forward(rows):
    """C5's gate and up (28672 x 8192 each, at least 64 rows a CU: the
    copy-staged kernel) plus a narrow weight through one qmm_forward_shared
    give each weight's own forward bits: the kernel is chosen per weight."""
    from swarmllm_amd import GgmlDType, fill_normal

    k = 8192
    mats = [QMatMul(QTensor.quantize(fill_normal(n * k, seed=90 + i, std=0.02).reshape(n, k), GgmlDType.Q4K))
            for i, n in enumerate((28672, 28672, 1024))]
    x = fill_normal(rows * k, seed=99).reshape(rows, k)
    shared = QMatMul.forward_shared(x, mats)
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))


# ---------------------------------------------------------------------------
# the Q6_K few-row matrix-core kernel: below k = 2048 every inner sum an exact
# int32, so the gap to the oracle is the order of the f32 scaling (~1e-7);
# from k = 2048 the weight enters as w8 = round(m_j (q - 32) / 256), one
# product a chunk, held to 1e-3 (the GEMM bound is 2e-3)
# ---------------------------------------------------------------------------
TIGHT_Q6K = 1e-5
ONE_Q6K = 1e-3


def q6k_skinny_bound(k):
    return ONE_Q6K if k >= 2048 else TIGHT_Q6K

Q6K_SKINNY_SHAPES = [  # (k, n, rows): past the 2 MiB line at 4-8 rows; rows of 3 and 5 super-blocks
    # (210-byte blocks at every 2-byte offset); ragged n; one and two 16-row tiles
    (4096, 2048, 4), (14336, 1000, 8), (2048, 1300, 6), (768, 700, 12), (1280, 513, 24),
    (256, 100, 9), (28672, 80, 16), (512, 129, 32),
]


def q6k(w: np.ndarray):
    wq = qref.from_float(qref.Q6_K, w)
    return QTensor.from_data(wq.tobytes(), w.shape, GgmlDType.Q6K, device=DEV), wq


@pytest.mark.parametrize("k,n,rows", Q6K_SKINNY_SHAPES)
def test_q6k_skinny_parity(k, n, rows):
    rng = np.random.default_rng(zlib.crc32(f"q6skinny-{k}-{n}-{rows}".encode()))
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = q6k(w)
    L = lib()
    before = L.qmm_gemm_launches()
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert L.qmm_gemm_launches() == before + 1, "the matrix-core kernel did not run"
    want = qref.matmul(qref.Q6_K, x, wq, n)
    wdeq = qref.to_float(qref.Q6_K, wq, n * k).reshape(n, k)
    err = normalised_error(y, want, wdeq, x)
    assert err <= q6k_skinny_bound(k), f"k={k} n={n} rows={rows}: {err}"


@pytest.mark.parametrize("rows", [8, 16])
def test_q6k_skinny_c5_down_projection(rows):
    """BASELINE C5's down projection (8192 x 28672 Q6_K) at the
    speculative-verification widths."""
    rng = np.random.default_rng(60 + rows)
    w = weights(rng, 8192, 28672)
    x = activations(rng, rows, 28672)
    qt, wq = q6k(w)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    kernel = lib().qmm_last_kernel().decode()
    assert "launch_q6" in kernel and "ONE = true" in kernel, kernel  # the single-product form
    want = qref.matmul(qref.Q6_K, x, wq, 8192)
    wdeq = qref.to_float(qref.Q6_K, wq, 8192 * 28672).reshape(8192, 28672)
    assert normalised_error(y, want, wdeq, x) <= ONE_Q6K


def test_q6k_skinny_shared_activation_equals_forward():
    """Q6_K weights through one qmm_forward_shared equal each weight's own
    forward bit for bit."""
    rng = np.random.default_rng(77)
    k = 2048
    mats = [QMatMul(q6k(weights(rng, n, k))[0]) for n in (1300, 100, 1500)]
    x = upload(activations(rng, 12, k))
    shared = QMatMul.forward_shared(x, mats)
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))


# ---------------------------------------------------------------------------
# the Q6_K GEMM (from 33 rows): 256 T_h + T_l is four times the reference's
# exact int32 super-block sum, so the gap to the oracle is again only the
# order of the f32 scaling
# ---------------------------------------------------------------------------
Q6K_GEMM_SHAPES = [  # (k, n, rows): one and many super-blocks; rows of 3, 5, 12 super-blocks (blocks at
    # every even offset of their windows) and of 8 and 56 (the same offset in every row); row and
    # weight-row tails; 4- and 8-wave tiles; the XCD remap (tiles % 8 == 0) and without it
    (256, 70, 33), (768, 300, 40), (1280, 129, 97), (2048, 64, 200), (3072, 4100, 129),
    (4096, 1000, 300), (14336, 256, 64), (2048, 2048, 512),
]


@pytest.mark.parametrize("k,n,rows", Q6K_GEMM_SHAPES)
def test_q6k_gemm_parity(k, n, rows):
    rng = np.random.default_rng(zlib.crc32(f"q6gemm-{k}-{n}-{rows}".encode()))
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = q6k(w)
    L = lib()
    before = L.qmm_gemm_launches()
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert L.qmm_gemm_launches() == before + 1, "the MFMA GEMM did not run"
    kernel = L.qmm_last_kernel().decode()
    single_pass = rows >= 129 and k % 2048 == 0
    assert ("launch_gemm_q6k_sp" if single_pass else "launch_gemm_q6k(") in kernel, kernel
    want = qref.matmul(qref.Q6_K, x, wq, n)
    wdeq = qref.to_float(qref.Q6_K, wq, n * k).reshape(n, k)
    err = normalised_error(y, want, wdeq, x)
    assert err <= TOL_GEMM, f"k={k} n={n} rows={rows}: {err}"
    assert err <= (TIGHT_SP if single_pass else TIGHT_Q6K), f"k={k} n={n} rows={rows}: {err}"


def test_q6k_gemm_special_activation_rows():
    """The quantizer's edge-case rows (zeros, a constant, one outlier, ties,
    subnormal values, one-signed runs, near powers of two), rows scaled by
    1e-30 and 1e30, against extreme group scales (a weight row with one
    large value per group)."""
    from helpers import special_rows

    k, n, rows = 2048, 96, 48
    rng = np.random.default_rng(92)
    w = weights(rng, n, k)
    w[5, ::16] = 3.0  # each group's scale -128 or 127 next to small codes
    w[6] = 0.0
    qt, wq = q6k(w)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    sp = special_rows(k)
    x[: len(sp)] = sp
    x[len(sp)] *= np.float32(1e-30)
    x[len(sp) + 1] *= np.float32(1e30)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert "launch_gemm_q6k(" in lib().qmm_last_kernel().decode()
    assert np.all(y[0] == 0.0) and np.all(y[:, 6] == 0.0)
    want = qref.matmul(qref.Q6_K, x, wq, n)
    wdeq = qref.to_float(qref.Q6_K, wq, n * k).reshape(n, k)
    assert normalised_error(y, want, wdeq, x) <= TIGHT_Q6K


def test_q6k_gemm_shared_activation_and_prequantized_equal_forward():
    """forward_shared over Q6_K weights and qmm_matmul from a quantized
    activation give each weight's own forward bit for bit at 64 rows."""
    from swarmllm_amd import _lib
    from swarmllm_amd.qtensor import quantize_act

    rng = np.random.default_rng(93)
    k = 1024
    mats = [QMatMul(q6k(weights(rng, n, k))[0]) for n in (300, 64, 1000)]
    x = upload(activations(rng, 64, k))
    shared = QMatMul.forward_shared(x, mats)
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))
    xq = quantize_act(x, _lib.ACT_Q8K)
    n = 300
    out = torch.empty((64, n), dtype=torch.float32, device=DEV)
    st = lib().qmm_matmul(qref.Q6_K, mats[0].qtensor.data_.data_ptr(), xq.data_ptr(), out.data_ptr(), n, k, n, 64,
                          torch.cuda.current_stream().cuda_stream)
    assert st == 0
    assert "launch_gemm_q6k(" in lib().qmm_last_kernel().decode()
    assert torch.equal(out, shared[0])


# ---------------------------------------------------------------------------
# Q6_K in one int8 pass (from 129 rows, k a multiple of 2048): the weight enters
# as round(m_j (q - 32) / 256) with m_j = round(127 sc_j / 16); held to 1e-3
# of ||w|| ||x|| (the 2e-3 bound)
# ---------------------------------------------------------------------------
Q6K_SP_SHAPES = [  # (k, n, rows): one and two row tiles, row and weight-row tails, cut along K and not
    (2048, 7, 129), (4096, 300, 256), (6144, 1000, 300), (14336, 200, 512), (2048, 4100, 383),
]


@pytest.mark.parametrize("k,n,rows", Q6K_SP_SHAPES)
def test_q6k_single_pass_gemm_parity(k, n, rows):
    rng = np.random.default_rng(zlib.crc32(f"q6sp-{k}-{n}-{rows}".encode()))
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = q6k(w)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert "launch_gemm_q6k_sp" in lib().qmm_last_kernel().decode()
    want = qref.matmul(qref.Q6_K, x, wq, n)
    wdeq = qref.to_float(qref.Q6_K, wq, n * k).reshape(n, k)
    err = normalised_error(y, want, wdeq, x)
    assert err <= TOL_GEMM
    assert err <= TIGHT_SP, f"k={k} n={n} rows={rows}: {err}"


def test_q6k_single_pass_gemm_extreme_scales_and_rows():
    """Weight rows with one large value per 16-value group (scales -128 and
    127 next to small codes, codes 0 and 63), a zero weight row; activation
    rows of the quantizer's edge cases and scaled by 1e-30, 1e-6, 1e3, 1e30."""
    from helpers import special_rows

    k, n, rows = 2048, 96, 160
    rng = np.random.default_rng(94)
    w = weights(rng, n, k)
    w[5, ::16] = 3.0
    w[7, ::16] = -3.0
    w[6] = 0.0
    qt, wq = q6k(w)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    sp = special_rows(k)
    x[: len(sp)] = sp
    for r, sc in zip(range(len(sp), len(sp) + 4), (1e-30, 1e-6, 1e3, 1e30)):
        x[r] *= np.float32(sc)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert "launch_gemm_q6k_sp" in lib().qmm_last_kernel().decode()
    assert np.all(y[0] == 0.0) and np.all(y[:, 6] == 0.0)
    want = qref.matmul(qref.Q6_K, x, wq, n)
    wdeq = qref.to_float(qref.Q6_K, wq, n * k).reshape(n, k)
    assert normalised_error(y, want, wdeq, x) <= TIGHT_SP


def test_q6k_single_pass_gemm_shared_and_prequantized():
    """Q6_K weights sharing an activation at 512 rows (one launch, each cut
    along K as its own forward cuts it) give each forward's bits, and forward
    is bit-identical run to run. Without a workspace for the cut (qmm_matmul
    from a quantized activation) a narrow Q6_K product runs on the exact
    kernel: within the single pass's bound of it."""
    from swarmllm_amd import _lib
    from swarmllm_amd.qtensor import quantize_act

    rng = np.random.default_rng(95)
    k, rows = 4096, 512
    mats = [QMatMul(q6k(weights(rng, n, k))[0]) for n in (1024, 300)]
    x = upload(activations(rng, rows, k, outliers=True))
    before = lib().qmm_gemm_launches()
    shared = QMatMul.forward_shared(x, mats)
    assert lib().qmm_gemm_launches() == before + 1
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))
        assert torch.equal(y, m.forward(x))
    xq = quantize_act(x, _lib.ACT_Q8K)
    n = 1024
    out = torch.empty((rows, n), dtype=torch.float32, device=DEV)
    assert lib().qmm_matmul(qref.Q6_K, mats[0].qtensor.data_.data_ptr(), xq.data_ptr(), out.data_ptr(), n, k, n, rows,
                            torch.cuda.current_stream().cuda_stream) == 0
    assert "launch_gemm_q6k(" in lib().qmm_last_kernel().decode()
    wdeq = mats[0].qtensor.dequantize().cpu().numpy()
    assert normalised_error(out.cpu().numpy(), shared[0].cpu().numpy(), wdeq, x.cpu().numpy()) <= TIGHT_SP


# ---------------------------------------------------------------------------
# the 32-value block formats (Q8_0, IQ4_NL, MXFP4) from 9 rows: one exact int32
# sum per block and output, scaled in f32 per block as the reference does
# ---------------------------------------------------------------------------
B32 = {"Q8_0": qref.Q8_0, "IQ4_NL": qref.IQ4_NL, "MXFP4": qref.MXFP4}
B32_SHAPES = [  # (k, n, rows): one block; a partial stage of 3 blocks; C4's 2880 (90 blocks, a partial last
    # stage); 4096; 129 blocks; row and weight-row tails; 4- and 8-wave tiles
    (32, 70, 9), (96, 33, 16), (2880, 300, 40), (4096, 1000, 129), (4128, 64, 200), (1024, 2048, 512),
]


def b32_weight(qtype, w: np.ndarray):
    wq = qref.from_float(qtype, w)
    return QTensor.from_data(wq.tobytes(), w.shape, GgmlDType(qtype), device=DEV), wq


@pytest.mark.parametrize("name", list(B32))
@pytest.mark.parametrize("k,n,rows", B32_SHAPES)
def test_b32_gemm_parity(name, k, n, rows):
    qtype = B32[name]
    rng = np.random.default_rng(zlib.crc32(f"b32gemm-{name}-{k}-{n}-{rows}".encode()))
    w = weights(rng, n, k)
    x = activations(rng, rows, k, outliers=True)
    qt, wq = b32_weight(qtype, w)
    L = lib()
    before = L.qmm_gemm_launches()
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert L.qmm_gemm_launches() == before + 1, "the MFMA GEMM did not run"
    assert "launch_gemm_b32(" in L.qmm_last_kernel().decode()
    want = qref.matmul(qtype, x, wq, n)
    wdeq = qref.to_float(qtype, wq, n * k).reshape(n, k)
    err = normalised_error(y, want, wdeq, x)
    assert err <= TOL_GEMM, f"{name} k={k} n={n} rows={rows}: {err}"
    assert err <= TIGHT_Q6K, f"{name} k={k} n={n} rows={rows}: {err}"  # exact block sums, f32 scaling


@pytest.mark.parametrize("name", list(B32))
def test_b32_gemm_special_rows(name):
    """The quantizer's edge-case activation rows, rows scaled by 1e-30 and
    1e5 (the f16 block scale of the activation overflows past about 8e6, in
    the reference as here), against a zero weight row and rows of large and
    tiny scales."""
    from helpers import special_rows

    qtype = B32[name]
    k, n, rows = 1024, 48, 24
    rng = np.random.default_rng(94)
    w = weights(rng, n, k)
    w[3] = 0.0
    w[4] *= np.float32(300.0)
    w[5] *= np.float32(1e-3)
    qt, wq = b32_weight(qtype, w)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    sp = special_rows(k)
    x[: len(sp)] = sp
    x[len(sp)] *= np.float32(1e-30)
    x[len(sp) + 1] *= np.float32(1e5)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    assert "launch_gemm_b32(" in lib().qmm_last_kernel().decode()
    assert np.all(y[0] == 0.0) and np.all(y[:, 3] == 0.0)
    want = qref.matmul(qtype, x, wq, n)
    wdeq = qref.to_float(qtype, wq, n * k).reshape(n, k)
    assert normalised_error(y, want, wdeq, x) <= TIGHT_Q6K


@pytest.mark.parametrize("name", list(B32))
def test_b32_gemm_shared_activation_and_prequantized_equal_forward(name):
    """forward_shared over 32-value weights and qmm_matmul from a quantized
    activation give each weight's own forward bit for bit at 20 rows."""
    from swarmllm_amd import _lib
    from swarmllm_amd.qtensor import quantize_act

    qtype = B32[name]
    rng = np.random.default_rng(95)
    k = 2880
    mats = [QMatMul(b32_weight(qtype, weights(rng, n, k))[0]) for n in (300, 64, 1000)]
    x = upload(activations(rng, 20, k))
    shared = QMatMul.forward_shared(x, mats)
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))
    xq = quantize_act(x, _lib.ACT_Q8_0)
    n = 300
    out = torch.empty((20, n), dtype=torch.float32, device=DEV)
    st = lib().qmm_matmul(qtype, mats[0].qtensor.data_.data_ptr(), xq.data_ptr(), out.data_ptr(), n, k, n, 20,
                          torch.cuda.current_stream().cuda_stream)
    assert st == 0
    assert "launch_gemm_b32(" in lib().qmm_last_kernel().decode()
    assert torch.equal(out, shared[0])
