"""Parity of the HIP path against the CPU oracle, through the C ABI.

Bit-exact: activation codes/scales/sums, weight quantization bytes,
dequantized values. Within tolerance (normalised by ||w_j||·||x_r||): the
products, 1e-3 for the decode/small-batch kernels.
"""
import ctypes
import zlib

import numpy as np
import pytest
import torch

from helpers import TOL_MATVEC, TYPES, normalised_error, special_rows, weights
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor, _lib
from swarmllm_amd._lib import lib
from swarmllm_amd.qtensor import act_planes, quantize_act

pytestmark = pytest.mark.gpu

DEV = "cuda"
TIGHT_MATVEC = 1e-5


def takes_matrix_cores(qtype, k, n, rows):
    """The library's few-rows policy (the reference's mmq_takes_few_rows,
    quantized/cuda.rs:790-839): Q4_K and Q6_K products of more than 8 rows,
    or of 4 and more on weights of 2 MiB and more, run on the int8 matrix
    cores."""
    if qtype not in (qref.Q4_K, qref.Q6_K):
        return False
    wbytes = n * (k // 256) * (144 if qtype == qref.Q4_K else 210)
    return rows > 8 or (rows >= 4 and wbytes >= 2 << 20)


def upload(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def qtensor_from_oracle(qtype: int, w: np.ndarray) -> tuple:
    wq = qref.from_float(qtype, w)
    return QTensor.from_data(wq.tobytes(), w.shape, GgmlDType(qtype), device=DEV), wq


# ---------------------------------------------------------------------------
# activation quantizers: bit-exact
# ---------------------------------------------------------------------------
def act_inputs(k: int, rows: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    sp = special_rows(k)
    x[: min(rows, len(sp))] = sp[: min(rows, len(sp))]
    return x


@pytest.mark.parametrize("k,rows", [(256, 1), (4096, 1), (14336, 3), (1024, 12)])
def test_q8k_activation_bit_exact(k, rows):
    x = act_inputs(k, rows, 1)
    x[-1, 7] = np.nan  # a NaN is never the block's largest; it codes as 127
    if k >= 768:
        # +inf and -inf both reach the block's |max|: the first decides the
        # sign; iscale is then -0, so inf * iscale is NaN (code 127) and d -inf
        x[-1, 256 + 3] = np.inf
        x[-1, 256 + 9] = -np.inf
        x[-1, 512 + 5] = -np.inf
    buf = quantize_act(upload(x), _lib.ACT_Q8K)
    codes, scales, sums = (t.cpu().numpy() for t in act_planes(buf, _lib.ACT_Q8K, k, rows))
    for r in range(rows):
        ref = qref.from_float(qref.Q8_K, x[r]).reshape(-1, 292)
        assert np.array_equal(codes[r].reshape(-1, 256), ref[:, 4:260].view(np.int8)), r
        assert np.array_equal(scales[r].view(np.uint32), ref[:, :4].copy().view(np.uint32).ravel()), r
        assert np.array_equal(sums[r].reshape(-1, 16), ref[:, 260:292].copy().view(np.int16)), r


@pytest.mark.parametrize("k,rows", [(32, 1), (2880, 1), (4096, 5), (14336, 2)])
def test_q8_0_activation_bit_exact(k, rows):
    x = act_inputs(k, rows, 2)
    x[-1, 5] = np.nan  # never the block's largest; `as i8` of NaN is 0
    if k >= 96:
        x[-1, 32 + 3] = np.inf  # amax inf: d inf, id 0, inf * 0 is NaN (code 0)
        x[-1, 64 + 7] = -np.inf
    buf = quantize_act(upload(x), _lib.ACT_Q8_0)
    codes, scales, sums = (t.cpu().numpy() for t in act_planes(buf, _lib.ACT_Q8_0, k, rows))
    for r in range(rows):
        ref = qref.from_float(qref.Q8_0, x[r]).reshape(-1, 34)
        rc = ref[:, 2:].view(np.int8)
        assert np.array_equal(codes[r].reshape(-1, 32), rc), r
        d16 = ref[:, :2].copy().view(np.float16).ravel()
        assert np.array_equal(scales[r], d16.astype(np.float32)), r
        assert np.array_equal(sums[r], rc.astype(np.int32).sum(1)), r


def test_strided_and_unaligned_activation_rows():
    k, rows = 512, 3
    x = np.random.default_rng(3).standard_normal((rows, k + 3)).astype(np.float32)
    xt = upload(x)
    L = lib()
    for layout in (_lib.ACT_Q8K, _lib.ACT_Q8_0):
        buf = torch.zeros(L.qmm_act_bytes(layout, k, rows), dtype=torch.uint8, device=DEV)
        # stride k+3 (not a multiple of 4) and a base 4 bytes past alignment
        st = L.qmm_quantize_act(xt.data_ptr() + 4, buf.data_ptr(), layout, k, rows, k + 3,
                                torch.cuda.current_stream().cuda_stream)
        assert st == 0
        codes = act_planes(buf, layout, k, rows)[0].cpu().numpy()
        vt = qref.Q8_K if layout == _lib.ACT_Q8K else qref.Q8_0
        for r in range(rows):
            ref = qref.from_float(vt, x[r, 1: 1 + k])
            if layout == _lib.ACT_Q8K:
                want = ref.reshape(-1, 292)[:, 4:260].view(np.int8).ravel()
            else:
                want = ref.reshape(-1, 34)[:, 2:].view(np.int8).ravel()
            assert np.array_equal(codes[r], want)


# ---------------------------------------------------------------------------
# weight quantizers (QTensor::quantize on the device) and dequantizers
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name", list(TYPES))
def test_weight_quantize_bit_exact(name):
    qtype = TYPES[name]
    k = 512
    rng = np.random.default_rng(4)
    w = np.concatenate([weights(rng, 64, k), special_rows(k), weights(rng, 8, k, std=3.0)]).astype(np.float32)
    q = QTensor.quantize(upload(w), GgmlDType(qtype))
    got = np.frombuffer(q.data(), np.uint8)
    want = qref.from_float(qtype, w)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{name}: {bad.size} bytes differ, first at {bad[:8]}"


def test_iq4_nl_zero_blocks_take_the_previous_levels():
    k = 256
    w = weights(np.random.default_rng(5), 4, k)
    w[1, 32:96] = 0.0     # two zero blocks after a non-zero one
    w[3, :] = 0.0         # a whole zero row
    w[0, :32] = 1e-16     # a first block below the 1e-15 threshold: no earlier levels
    q = QTensor.quantize(upload(w), GgmlDType.Iq4Nl)
    assert np.array_equal(np.frombuffer(q.data(), np.uint8), qref.from_float(qref.IQ4_NL, w))


def test_mxfp4_exponents_near_powers_of_two():
    p = np.float32(2.0) ** np.arange(-20, 20, dtype=np.float32)
    vals = []
    for v in p:
        x = v
        for _ in range(40):
            x = np.nextafter(x, np.float32(0))
            vals.append(x)
        vals.append(v)
        x = v
        for _ in range(20):
            x = np.nextafter(x, np.float32(np.inf))
            vals.append(x)
    amaxes = np.array(vals, dtype=np.float32)
    w = np.zeros((amaxes.size, 32), np.float32)
    w[:, 0] = amaxes
    w[:, 1:] = amaxes[:, None] * np.float32(0.3)
    w = w.reshape(-1)[: (w.size // 32) * 32]
    q = QTensor.quantize(upload(w.reshape(1, -1)), GgmlDType.Mxfp4)
    assert np.array_equal(np.frombuffer(q.data(), np.uint8), qref.from_float(qref.MXFP4, w))


@pytest.mark.parametrize("name", list(TYPES))
def test_dequantize_bit_exact(name):
    qtype = TYPES[name]
    k = 1024
    w = np.concatenate([weights(np.random.default_rng(6), 16, k), special_rows(k)])
    qt, wq = qtensor_from_oracle(qtype, w)
    got = qt.dequantize().cpu().numpy()
    want = qref.to_float(qtype, wq, w.size).reshape(w.shape)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    f16 = qt.dequantize_f16().cpu().numpy()
    assert np.array_equal(f16.view(np.uint16), want.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------
# products: decode (1 row) and small batches (2..8 rows), then the rest
# ---------------------------------------------------------------------------
SHAPES = {
    "Q4_K": [(256, 7), (1024, 96), (4096, 1029), (14336, 64)],
    "Q6_K": [(256, 5), (1024, 96), (4096, 515), (14336, 33), (512, 64)],
    "Q8_0": [(32, 3), (96, 17), (4096, 300), (2880, 77), (8224, 9)],
    "IQ4_NL": [(32, 3), (4096, 129), (2880, 40), (160, 64)],
    "MXFP4": [(32, 2), (2880, 133), (4096, 64), (8224, 5)],
}


def case_list():
    out = []
    for name, shapes in SHAPES.items():
        for k, n in shapes:
            for rows in (1, 2, 3, 5, 8):
                out.append((name, k, n, rows))
    return out


@pytest.mark.parametrize("name,k,n,rows", case_list())
def test_matvec_parity(name, k, n, rows):
    qtype = TYPES[name]
    rng = np.random.default_rng(zlib.crc32(f"{name}-{k}-{n}-{rows}".encode()))
    w = weights(rng, n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    qt, wq = qtensor_from_oracle(qtype, w)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    want = qref.matmul(qtype, x, wq, n)
    wdeq = qref.to_float(qtype, wq, n * k).reshape(n, k)
    err = normalised_error(y, want, wdeq, x)
    assert err <= TOL_MATVEC, f"{name} k={k} n={n} rows={rows}: {err}"
    if takes_matrix_cores(qtype, k, n, rows):
        # the few-rows matrix-core products (test_gemm_gpu.py covers them)
        assert err <= 5e-4, f"{name} k={k} n={n} rows={rows}: {err}"
        return
    # Both sides sum the same exact int32 block products and differ only in
    # the order of their f32 scaling, so the gap is f32 rounding (~1e-7);
    # a dropped or misindexed block term shows up far above this bound.
    assert err <= TIGHT_MATVEC, f"{name} k={k} n={n} rows={rows}: {err}"


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows", [9, 16, 21])
def test_forward_beyond_the_matvec_rows(name, rows):
    qtype = TYPES[name]
    k, n = (512, 70) if qtype in (12, 14) else (2880, 70)
    rng = np.random.default_rng(rows)
    w = weights(rng, n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    qt, wq = qtensor_from_oracle(qtype, w)
    y = QMatMul(qt).forward(upload(x)).cpu().numpy()
    want = qref.matmul(qtype, x, wq, n)
    wdeq = qref.to_float(qtype, wq, n * k).reshape(n, k)
    assert normalised_error(y, want, wdeq, x) <= TOL_MATVEC


def test_forward_shape_rules():
    """cpu_fwd's shape rules (mod.rs:1280-1333): leading dims kept, k checked,
    contiguity required."""
    k, n = 512, 40
    rng = np.random.default_rng(8)
    qt, _ = qtensor_from_oracle(qref.Q4_K, weights(rng, n, k))
    mm = QMatMul(qt)
    x = upload(rng.standard_normal((2, 3, k)).astype(np.float32))
    y = mm.forward(x)
    assert tuple(y.shape) == (2, 3, n)
    with pytest.raises(ValueError):
        mm.forward(upload(np.zeros((1, k + 32), np.float32)))
    with pytest.raises(ValueError):
        mm.forward(x.transpose(0, 1))


@pytest.mark.parametrize("name", list(TYPES))
def test_batch_invariance(name):
    """A row's result does not depend on the rows beside it, for every batch
    width up to 8 (the reference's qmm_batch, quantized_tests.rs:223-258,
    which asserts exact equality within its one-to-eight-row kernel). From 9
    rows every type runs on the matrix cores, whose f32 scaling is ordered
    differently (test_gemm_gpu.py covers those widths)."""
    qtype = TYPES[name]
    k, n = (4096, 70) if qtype in (12, 14) else (2880, 70)
    rng = np.random.default_rng(80 + qtype)
    qt, _ = qtensor_from_oracle(qtype, weights(rng, n, k))
    mm = QMatMul(qt)
    xs = upload(rng.standard_normal((12, k)).astype(np.float32))
    alone = mm.forward(xs[:1].contiguous())
    widths = (2, 3, 4, 5, 6, 7, 8)
    for rows in widths:
        y = mm.forward(xs[:rows].contiguous())
        assert torch.equal(y[0], alone[0]), rows


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("rows", [1, 2, 3])
def test_forward_shared_equals_forward(name, rows):
    """forward_shared (qmm_forward_shared) returns what each weight's own
    forward returns, bit for bit: more weights than one launch takes (6 > 4),
    ragged row counts, odd ones."""
    qtype = TYPES[name]
    k = 1024 if qtype in (12, 14) else 2880
    rng = np.random.default_rng(9 + rows)
    mats = [QMatMul(qtensor_from_oracle(qtype, weights(rng, n, k))[0]) for n in (96, 32, 33, 1, 160, 7)]
    x = upload(rng.standard_normal((rows, k)).astype(np.float32))
    shared = QMatMul.forward_shared(x, mats)
    for m, y in zip(mats, shared):
        assert torch.equal(y, m.forward(x))


# (two rows stream, and quantize in the kernel, up to k = 8192)
@pytest.mark.parametrize("k,rows", [(k, 1) for k in (256, 1024, 4096, 8192, 14336, 16384)] +
                         [(k, 2) for k in (256, 1024, 4096, 8192)])
def test_q4k_in_kernel_quantization_matches_standalone(k, rows):
    """The decode kernel quantizing its activation in LDS gives the same bits
    as the same kernel reading the standalone quantizer's planes (which are
    bit-exact to BlockQ8K::from_float): the in-kernel quantization is that
    quantization. Also within tolerance of the oracle."""
    n = 300
    rng = np.random.default_rng(k + rows)
    w = weights(rng, n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[0, :256] = special_rows(256)[3]  # ties in |x| of both signs
    qt, wq = qtensor_from_oracle(qref.Q4_K, w)
    xt = upload(x)
    fused = QMatMul(qt).forward(xt)
    L = lib()
    xq = quantize_act(xt, _lib.ACT_Q8K)
    pre = torch.empty((rows, n), dtype=torch.float32, device=DEV)
    st = L.qmm_matvec(qref.Q4_K, qt.data_.data_ptr(), xq.data_ptr(), pre.data_ptr(), n, k, n, rows,
                      torch.cuda.current_stream().cuda_stream)
    assert st == 0
    assert torch.equal(fused, pre)
    want = qref.matmul(qref.Q4_K, x, wq, n)
    wdeq = qref.to_float(qref.Q4_K, wq, n * k).reshape(n, k)
    assert normalised_error(fused.cpu().numpy(), want, wdeq, x) <= TOL_MATVEC


def test_q4k_unaligned_activation_takes_the_quantize_then_product_path():
    """An activation that is not 16-byte aligned goes through the standalone
    quantizer and the same product kernel: the same bits as aligned."""
    k, n = 1024, 64
    rng = np.random.default_rng(11)
    qt, _ = qtensor_from_oracle(qref.Q4_K, weights(rng, n, k))
    x = rng.standard_normal((1, k)).astype(np.float32)
    base = upload(np.concatenate([np.zeros(1, np.float32), x.ravel()]))
    xs = base[1:].reshape(1, k)  # 4 bytes past the allocation's alignment
    assert xs.data_ptr() % 16 == 4
    y_unaligned = QMatMul(qt).forward(xs)
    y_aligned = QMatMul(qt).forward(upload(x))
    assert torch.equal(y_unaligned, y_aligned)


def test_full_size_decode_gate_projection():
    """C2's headline product at full size (Q4_K 14336 x 4096, M = 1), the
    weight quantized on the device: against the oracle on the same bytes."""
    n, k = 14336, 4096
    from swarmllm_amd import fill_normal
    w = fill_normal(n * k, seed=1, std=0.02).reshape(n, k)
    x = fill_normal(k, seed=101).reshape(1, k)
    qt = QTensor.quantize(w, GgmlDType.Q4K)
    y = QMatMul(qt).forward(x).cpu().numpy()
    wq = np.frombuffer(qt.data(), np.uint8)
    xn = x.cpu().numpy()
    want = qref.matmul(qref.Q4_K, xn, wq, n)
    wdeq = qt.dequantize().cpu().numpy()
    assert normalised_error(y, want, wdeq, xn) <= TOL_MATVEC
    # the device quantizer agrees with the oracle's on a slice of the weight
    sl = w[:64].cpu().numpy()
    assert np.array_equal(wq[: 64 * 16 * 144], qref.from_float(qref.Q4_K, sl))


def test_status_paths_on_device():
    k, n = 256, 8
    qt, _ = qtensor_from_oracle(qref.Q4_K, weights(np.random.default_rng(10), n, k))
    x = upload(np.ones((1, k), np.float32))
    out = torch.empty((1, n), dtype=torch.float32, device=DEV)
    L = lib()
    need = ctypes.c_size_t(0)
    st = torch.cuda.current_stream().cuda_stream
    assert L.qmm_forward(12, qt.data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n, None, 0, ctypes.byref(need),
                         k, n, 1, 0, st) == 0
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    small = torch.empty(need.value - 1, dtype=torch.uint8, device=DEV)
    assert L.qmm_forward(12, qt.data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n, small.data_ptr(),
                         small.numel(), ctypes.byref(need), k, n, 1, 1, st) == _lib.QMM_WORKSPACE_TOO_SMALL
    before = L.qmm_matvec_launches()
    L.qmm_fail_next_launch()
    assert L.qmm_forward(12, qt.data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n, ws.data_ptr(), ws.numel(),
                         ctypes.byref(need), k, n, 1, 1, st) == _lib.QMM_NO_ROOM
    assert L.qmm_matvec_launches() == before
    assert L.qmm_forward(12, qt.data_.data_ptr(), x.data_ptr(), k, out.data_ptr(), n, ws.data_ptr(), ws.numel(),
                         ctypes.byref(need), k, n, 1, 1, st) == 0
    assert L.qmm_matvec_launches() == before + 1
    assert L.qmm_available() == 1
