"""Grouped expert products (qmm_moe_forward, the reference's moe_gemm_gguf /
QMatMul::matmul_many) against the CPU oracle, through the C ABI, for the
32-value formats (MXFP4, Q8_0, IQ4_NL) and the K-quants (Q4_K, Q6_K).

Routing as BASELINE C4 draws it: N(0,1) router logits [tokens, experts],
top-k per token with ties to the lower index, routing entries sorted by
(expert, pair), pair = token * topk + choice, routing weights the softmax of
the chosen logits. Each product is checked against the oracle's matmul of
that pair's input row and expert weight (normalised error <= 1e-3, the decode
bound) and must equal qmm_forward of the same pair times its scale bit for
bit (matmul_many == per-job forward, quantized/mod.rs:743-745).
"""
import ctypes
import zlib

import numpy as np
import pytest
import torch

from helpers import TOL_MATVEC, normalised_error
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal, moe_forward
from swarmllm_amd._lib import QMM_NO_ROOM, QMM_UNSUPPORTED, QMM_WORKSPACE_TOO_SMALL, lib

pytestmark = pytest.mark.gpu

DEV = "cuda"
MOE_TYPES = {"MXFP4": 39, "Q8_0": 8, "IQ4_NL": 20, "Q4_K": 12, "Q6_K": 14}
KQUANT = {12, 14}


def routing(tokens: int, experts: int, topk: int, seed: int):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    choice = np.argsort(-logits, axis=1, kind="stable")[:, :topk]
    pairs = sorted((int(choice[t, j]), t * topk + j) for t in range(tokens) for j in range(topk))
    expert_ids = np.array([e for e, _ in pairs], np.int32)
    sorted_ids = np.array([p for _, p in pairs], np.int32)
    sel = np.take_along_axis(logits, choice, axis=1).astype(np.float64)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    return sorted_ids, expert_ids, w.reshape(-1).astype(np.float32)


def expert_stack(qtype: int, e: int, n: int, k: int, seed: int) -> QTensor:
    """E experts [n, k] quantized on the device (bit-exact to from_float), stacked."""
    parts = [QTensor.quantize(fill_normal(n * k, seed=(seed << 8) | i, std=0.02).reshape(n, k), GgmlDType(qtype))
             for i in range(e)]
    return QTensor(torch.cat([p.data_ for p in parts]), (e, n, k), GgmlDType(qtype))


def t32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def check_against_oracle(qtype, stack, x, out, sorted_ids, expert_ids, topk_w, topk):
    e, n, k = stack.shape
    wb = stack.data_.cpu().numpy()
    per = wb.size // e
    for i in range(len(sorted_ids)):
        p, ex = int(sorted_ids[i]), int(expert_ids[i])
        row = p if topk_w is not None else p // topk
        scale = np.float32(topk_w[p]) if topk_w is not None else np.float32(1.0)
        w_e = wb[ex * per:(ex + 1) * per]
        want = qref.matmul(qtype, x[row][None, :], w_e, n)[0] * scale
        wdeq = qref.to_float(qtype, w_e, n * k).reshape(n, k)
        err = normalised_error(out[p][None, :], want[None, :], wdeq, (x[row] * scale)[None, :])
        assert err <= TOL_MATVEC, f"pair {p} expert {ex}: {err}"


def check_against_forward(stack, xs_dev, out, sorted_ids, expert_ids, topk_w, topk):
    e, n, k = stack.shape
    per = stack.data_.numel() // e
    for i in range(len(sorted_ids)):
        p, ex = int(sorted_ids[i]), int(expert_ids[i])
        row = p if topk_w is not None else p // topk
        qt = QTensor(stack.data_[ex * per:(ex + 1) * per], (n, k), stack.dtype)
        y = QMatMul(qt).forward(xs_dev[row:row + 1]).cpu().numpy()[0]
        scale = np.float32(topk_w[p]) if topk_w is not None else np.float32(1.0)
        assert np.array_equal((y * scale).view(np.uint32), out[p].view(np.uint32)), f"pair {p}"


@pytest.mark.parametrize("name", list(MOE_TYPES))
@pytest.mark.parametrize("weighted", [False, True])
def test_moe_parity_small(name, weighted):
    qtype = MOE_TYPES[name]
    E, n, tokens, topk = 8, 96, 6, 3
    k = 512 if qtype in KQUANT else 320
    seed = zlib.crc32(f"{name}-{weighted}".encode())
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, seed)
    stack = expert_stack(qtype, E, n, k, seed & 0xFFFF)
    rows = tokens * topk if weighted else tokens
    x = np.random.default_rng(seed).standard_normal((rows, k)).astype(np.float32)
    xs = t32(x)
    tw = topk_w if weighted else None
    out = moe_forward(xs, stack, t32(sorted_ids), t32(expert_ids), t32(topk_w) if weighted else None, topk)
    out = out.cpu().numpy()
    check_against_oracle(qtype, stack, x, out, sorted_ids, expert_ids, tw, topk)
    check_against_forward(stack, xs, out, sorted_ids, expert_ids, tw, topk)


def test_moe_c4_gpt_oss_shapes():
    """BASELINE C4: 32 MXFP4 experts, gate_up [5760, 2880] then down
    [2880, 2880], 8 tokens with top-4 routing."""
    qtype, E, tokens, topk = 39, 32, 8, 4
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, 4)
    before = lib().qmm_moe_launches()
    gate_up = expert_stack(qtype, E, 5760, 2880, 41)
    x = np.random.default_rng(40).standard_normal((tokens, 2880)).astype(np.float32)
    xs = t32(x)
    y1 = moe_forward(xs, gate_up, t32(sorted_ids), t32(expert_ids), None, topk).cpu().numpy()
    check_against_oracle(qtype, gate_up, x, y1, sorted_ids, expert_ids, None, topk)
    check_against_forward(gate_up, xs, y1, sorted_ids, expert_ids, None, topk)
    del gate_up
    down = expert_stack(qtype, E, 2880, 2880, 42)
    x2 = np.random.default_rng(43).standard_normal((tokens * topk, 2880)).astype(np.float32)
    xs2 = t32(x2)
    y2 = moe_forward(xs2, down, t32(sorted_ids), t32(expert_ids), t32(topk_w), topk).cpu().numpy()
    check_against_oracle(qtype, down, x2, y2, sorted_ids, expert_ids, topk_w, topk)
    check_against_forward(down, xs2, y2, sorted_ids, expert_ids, topk_w, topk)
    assert lib().qmm_moe_launches() >= before + 2


@pytest.mark.parametrize("name", ["MXFP4", "Q8_0", "IQ4_NL"])
@pytest.mark.parametrize("k", [2048, 2880, 4032])
def test_moe_packed_lane_rows(name, k):
    """Rows of 64-126 blocks, an even number, take the packed form (each lane
    a two-block unit of the wave's contiguous rows, whichever row it falls
    in; MXFP4 takes the matrix-core form); each entry must still equal
    qmm_forward of its pair bit for bit.
    n = 203 leaves the last workgroup and the last wave partly empty, and the
    routing gives runs of one to several entries."""
    qtype = MOE_TYPES[name]
    E, n, tokens, topk = 5, 203, 7, 3
    seed = zlib.crc32(f"packed-{name}-{k}".encode())
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, seed)
    stack = expert_stack(qtype, E, n, k, seed & 0xFFFF)
    for weighted in (False, True):
        rows = tokens * topk if weighted else tokens
        x = np.random.default_rng(seed + weighted).standard_normal((rows, k)).astype(np.float32)
        xs = t32(x)
        tw = topk_w if weighted else None
        out = moe_forward(xs, stack, t32(sorted_ids), t32(expert_ids), t32(topk_w) if weighted else None, topk)
        out = out.cpu().numpy()
        check_against_oracle(qtype, stack, x, out, sorted_ids, expert_ids, tw, topk)
        check_against_forward(stack, xs, out, sorted_ids, expert_ids, tw, topk)


@pytest.mark.parametrize("k", [32, 96, 1056, 2880, 4096])
def test_moe_fp4_matrix_core_rows(k):
    """MXFP4 rows of up to 128 blocks take the matrix-core form (block sums
    on v_mfma_scale_f32_16x16x128_f8f6f4, the codes split as 16 h + l): one
    block, odd block counts (a group of four blocks partly past the row), the
    128-block maximum; a run of 10 entries (three passes of up to 4), n = 203
    (the last wave's 16 columns partly past the rows). A routing this small
    takes the one-launch form, the kernel quantizing its input rows and
    finding the runs itself. Each entry must equal qmm_forward of its pair
    bit for bit (the two-launch form of larger routings is checked the same
    way in test_moe_prepass_form_matches_one_launch_form)."""
    qtype = MOE_TYPES["MXFP4"]
    E, n, tokens, topk = 3, 203, 10, 2
    seed = zlib.crc32(f"fp4-mc-{k}".encode())
    rng = np.random.default_rng(seed)
    # expert 1 takes every token's first choice: a run of 10 entries
    pairs = sorted((1 if j == 0 else (0, 2)[int(rng.integers(2))], t * topk + j)
                   for t in range(tokens) for j in range(topk))
    expert_ids = np.array([e for e, _ in pairs], np.int32)
    sorted_ids = np.array([p for _, p in pairs], np.int32)
    topk_w = rng.random(tokens * topk).astype(np.float32)
    stack = expert_stack(qtype, E, n, k, seed & 0xFFFF)
    for weighted in (False, True):
        rows = tokens * topk if weighted else tokens
        x = rng.standard_normal((rows, k)).astype(np.float32)
        xs = t32(x)
        tw = topk_w if weighted else None
        out = moe_forward(xs, stack, t32(sorted_ids), t32(expert_ids), t32(topk_w) if weighted else None, topk)
        assert "launch_moe_fp4_fused" in lib().qmm_last_kernel().decode()
        out = out.cpu().numpy()
        check_against_oracle(qtype, stack, x, out, sorted_ids, expert_ids, tw, topk)
        check_against_forward(stack, xs, out, sorted_ids, expert_ids, tw, topk)


@pytest.mark.parametrize("size_m", [256, 257])
def test_moe_fp4_one_launch_boundary(size_m):
    """MXFP4 routings of up to 256 entries take the one-launch form (the
    kernel quantizing its input rows and finding the runs), 257 and more the
    quantizing launch and its run table; on both sides of the line every
    entry equals qmm_forward of its pair bit for bit, with per-pair inputs
    and routing weights (2880-value rows, runs of many entries)."""
    qtype = MOE_TYPES["MXFP4"]
    E, n, k, topk = 6, 48, 2880, 1
    sorted_ids, expert_ids, topk_w = routing(size_m, E, topk, 257 + size_m)
    stack = expert_stack(qtype, E, n, k, size_m)
    x = np.random.default_rng(size_m).standard_normal((size_m, k)).astype(np.float32)
    xs = t32(x)
    out = moe_forward(xs, stack, t32(sorted_ids), t32(expert_ids), t32(topk_w), topk)
    kernel = lib().qmm_last_kernel().decode()
    assert ("launch_moe_fp4_fused" in kernel) == (size_m <= 256) and "launch_moe_fp4" in kernel, kernel
    out = out.cpu().numpy()
    check_against_forward(stack, xs, out, sorted_ids, expert_ids, topk_w, topk)
    sel = slice(0, size_m, 16)
    check_against_oracle(qtype, stack, x, out, sorted_ids[sel], expert_ids[sel], topk_w, topk)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("size_m", [256, 257])
def test_moe_kq_one_launch_boundary(name, size_m):
    """Q4_K and Q6_K routings of up to 256 entries take the one-launch form
    (the kernel quantizing its input rows to Q8_K in LDS and finding the
    runs), larger ones the quantizing launch and its run table; on both sides
    every entry equals qmm_forward of its pair bit for bit."""
    qtype = MOE_TYPES[name]
    E, n, k, topk = 6, 48, 2048, 1
    sorted_ids, expert_ids, topk_w = routing(size_m, E, topk, 911 + size_m)
    stack = expert_stack(qtype, E, n, k, 3 * size_m)
    x = np.random.default_rng(size_m + 5).standard_normal((size_m, k)).astype(np.float32)
    xs = t32(x)
    out = moe_forward(xs, stack, t32(sorted_ids), t32(expert_ids), t32(topk_w), topk)
    kernel = lib().qmm_last_kernel().decode()
    assert ("kFused = true" in kernel) == (size_m <= 256), kernel
    out = out.cpu().numpy()
    check_against_forward(stack, xs, out, sorted_ids, expert_ids, topk_w, topk)
    sel = slice(0, size_m, 16)
    check_against_oracle(qtype, stack, x, out, sorted_ids[sel], expert_ids[sel], topk_w, topk)


def moe_into(stack, xs, x_stride, sorted_ids, expert_ids, topk_w, topk, rows_out, fill=float("nan")):
    """qmm_moe_forward through the C ABI into an output prefilled with `fill`
    (rows the routing does not reach keep it)."""
    L = lib()
    e, n, k = stack.shape
    size_m = len(sorted_ids)
    out = torch.full((rows_out, n), fill, dtype=torch.float32, device=DEV)
    sid, eid = t32(sorted_ids), t32(expert_ids)
    tw = t32(topk_w) if topk_w is not None else None
    need = ctypes.c_size_t(0)
    args = (int(stack.dtype), stack.data_.data_ptr(), e, xs.data_ptr(), x_stride, sid.data_ptr(), eid.data_ptr(),
            tw.data_ptr() if tw is not None else None, topk, out.data_ptr(), n)
    assert L.qmm_moe_forward(*args, None, 0, ctypes.byref(need), k, n, size_m, 0, 0) == 0
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=DEV)
    assert L.qmm_moe_forward(*args, ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, size_m, 1, 0) == 0
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("k", [256, 2880])  # MXFP4 (type 39): the matrix-core form
def test_moe_order_of_entries_does_not_change_results(k):
    """Any order of the routing entries gives the same bits; out of expert
    order there are more runs than experts, and every one is computed (the
    output starts as NaN, so a run left out shows)."""
    qtype, E, n, tokens, topk = 39, 6, 64, 5, 2
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, 7)
    stack = expert_stack(qtype, E, n, k, 77)
    xs = t32(np.random.default_rng(7).standard_normal((tokens, k)).astype(np.float32))
    ref = moe_into(stack, xs, k, sorted_ids, expert_ids, None, topk, tokens * topk)
    assert not np.isnan(ref).any()
    perm = np.random.default_rng(8).permutation(len(sorted_ids))
    runs = 1 + int(np.count_nonzero(np.diff(expert_ids[perm])))
    assert runs > E
    got = moe_into(stack, xs, k, sorted_ids[perm], expert_ids[perm], None, topk, tokens * topk)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("k", [128, 2048])  # 2048: the packed form
def test_moe_more_runs_than_experts(k):
    """Entries alternating between two experts: six runs over two experts."""
    qtype, E, n, topk = 8, 2, 48, 1
    stack = expert_stack(qtype, E, n, k, 13)
    x = np.random.default_rng(13).standard_normal((6, k)).astype(np.float32)
    xs = t32(x)
    sorted_ids = np.arange(6, dtype=np.int32)
    expert_ids = np.array([0, 1, 0, 1, 0, 1], np.int32)
    got = moe_into(stack, xs, k, sorted_ids, expert_ids, None, topk, 6)
    check_against_oracle(qtype, stack, x, got, sorted_ids, expert_ids, None, topk)
    check_against_forward(stack, xs, got, sorted_ids, expert_ids, None, topk)


@pytest.mark.parametrize("name", ["MXFP4", "Q8_0", "Q4_K", "Q6_K"])
def test_moe_prepass_form_matches_one_launch_form(name):
    """Routings above a decode step's size, and inputs whose rows are not
    16-byte aligned, take the runs pre-pass and the standalone quantizer;
    both forms give the same bits, and the large routing matches the oracle
    and qmm_forward."""
    qtype = MOE_TYPES[name]
    E, n, k, topk = 8, 64, 256, 4
    tokens = 80  # 320 routing entries
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, 21)
    stack = expert_stack(qtype, E, n, k, 21)
    x = np.random.default_rng(21).standard_normal((tokens * topk, k)).astype(np.float32)
    xs = t32(x)
    big = moe_into(stack, xs, k, sorted_ids, expert_ids, topk_w, topk, tokens * topk)
    assert not np.isnan(big).any()
    check_against_forward(stack, xs, big, sorted_ids, expert_ids, topk_w, topk)
    sel = slice(0, len(sorted_ids), 7)
    check_against_oracle(qtype, stack, x, big, sorted_ids[sel], expert_ids[sel], topk_w, topk)
    # a decode-sized routing: the one-launch form, then the same inputs at a
    # row stride of k + 1 floats (rows not 16-byte aligned): the pre-pass form
    sid, eid, tw = routing(6, E, topk, 22)
    x6 = np.random.default_rng(22).standard_normal((6 * topk, k)).astype(np.float32)
    one = moe_into(stack, t32(x6), k, sid, eid, tw, topk, 6 * topk)
    padded = np.zeros((6 * topk, k + 1), np.float32)
    padded[:, :k] = x6
    two = moe_into(stack, t32(padded), k + 1, sid, eid, tw, topk, 6 * topk)
    assert not np.isnan(one).any()
    assert np.array_equal(one.view(np.uint32), two.view(np.uint32))


@pytest.mark.parametrize("k", [64, 2880])  # MXFP4 (type 39): the matrix-core form
def test_moe_out_of_range_entries_write_nothing(k):
    qtype, E, n, topk = 39, 4, 32, 1
    stack = expert_stack(qtype, E, n, k, 9)
    x = np.random.default_rng(9).standard_normal((6, k)).astype(np.float32)
    sorted_ids = np.array([0, 1, 2, 3, 4, 5], np.int32)
    expert_ids = np.array([-1, 0, 0, 2, 4, 7], np.int32)  # -1, 4 and 7 are not experts
    L = lib()
    out = torch.full((6, n), 123.5, dtype=torch.float32, device=DEV)
    xs, sid, eid = t32(x), t32(sorted_ids), t32(expert_ids)
    need = ctypes.c_size_t(0)
    args = (qtype, stack.data_.data_ptr(), E, xs.data_ptr(), k, sid.data_ptr(), eid.data_ptr(), None, topk,
            out.data_ptr(), n)
    assert L.qmm_moe_forward(*args, None, 0, ctypes.byref(need), k, n, 6, 0, 0) == 0
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    assert L.qmm_moe_forward(*args, ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, 6, 1, 0) == 0
    got = out.cpu().numpy()
    for p in (0, 4, 5):
        assert np.all(got[p] == 123.5), f"row {p} was written"
    check_against_forward(stack, xs, got, sorted_ids[1:4], expert_ids[1:4], None, topk)


def test_moe_status_paths():
    qtype, E, n, k, topk = 39, 2, 32, 64, 2
    stack = expert_stack(qtype, E, n, k, 11)
    x = torch.zeros((2, k), dtype=torch.float32, device=DEV)
    sid = t32(np.array([0, 1, 2, 3], np.int32))
    eid = t32(np.array([0, 0, 1, 1], np.int32))
    out = torch.empty((4, n), dtype=torch.float32, device=DEV)
    L = lib()
    need = ctypes.c_size_t(0)
    args = (qtype, stack.data_.data_ptr(), E, x.data_ptr(), k, sid.data_ptr(), eid.data_ptr(), None, topk,
            out.data_ptr(), n)
    assert L.qmm_moe_forward(*args, None, 0, ctypes.byref(need), k, n, 4, 0, 0) == 0 and need.value > 0
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    assert L.qmm_moe_forward(*args, ws.data_ptr(), need.value - 1, ctypes.byref(need), k, n, 4, 1, 0) == \
        QMM_WORKSPACE_TOO_SMALL
    L.qmm_fail_next_launch()
    assert L.qmm_moe_forward(*args, ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, 4, 1, 0) == QMM_NO_ROOM
    assert L.qmm_moe_forward(*args, ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, 4, 1, 0) == 0
    # per-token inputs need size_m to be a multiple of topk; K-quant rows of
    # more than 16384 values are not a grouped shape here
    assert L.qmm_moe_forward(*args, ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, 3, 1, 0) == QMM_UNSUPPORTED
    for t in (12, 14):
        args_kq = (t,) + args[1:]
        assert L.qmm_moe_forward(*args_kq, None, 0, ctypes.byref(need), 16640, n, 4, 0, 0) == QMM_UNSUPPORTED


def test_moe_kquant_qwen3_moe_like_shapes():
    """Q4_K gate [768, 2048] and Q6_K down [2048, 768] over 128 experts,
    4 tokens with top-8 routing (the expert shapes of a Qwen3-MoE layer):
    every pair against the oracle and bit-identical to its qmm_forward."""
    E, tokens, topk = 128, 4, 8
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, 31)
    before = lib().qmm_moe_launches()
    gate = expert_stack(12, E, 768, 2048, 31)
    x = np.random.default_rng(31).standard_normal((tokens, 2048)).astype(np.float32)
    xs = t32(x)
    y1 = moe_forward(xs, gate, t32(sorted_ids), t32(expert_ids), None, topk).cpu().numpy()
    check_against_oracle(12, gate, x, y1, sorted_ids, expert_ids, None, topk)
    check_against_forward(gate, xs, y1, sorted_ids, expert_ids, None, topk)
    del gate
    down = expert_stack(14, E, 2048, 768, 32)
    x2 = np.random.default_rng(32).standard_normal((tokens * topk, 768)).astype(np.float32)
    xs2 = t32(x2)
    y2 = moe_forward(xs2, down, t32(sorted_ids), t32(expert_ids), t32(topk_w), topk).cpu().numpy()
    check_against_oracle(14, down, x2, y2, sorted_ids, expert_ids, topk_w, topk)
    check_against_forward(down, xs2, y2, sorted_ids, expert_ids, topk_w, topk)
    assert lib().qmm_moe_launches() >= before + 2


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("k", [4352, 8448, 16384])
def test_moe_kquant_long_rows(name, k):
    """Rows past 16 super-blocks (Q4_K: two and four units a lane; Q6_K:
    two and more spans), and at 16384 values fewer entries a chunk than the
    run holds (the chunk's rows fill the LDS budget): 7 entries on one
    expert, 2 on another."""
    qtype = MOE_TYPES[name]
    E, n, topk = 3, 40, 1
    stack = expert_stack(qtype, E, n, k, k + qtype)
    x = np.random.default_rng(k).standard_normal((9, k)).astype(np.float32)
    xs = t32(x)
    sorted_ids = np.arange(9, dtype=np.int32)
    expert_ids = np.array([1] * 7 + [2] * 2, np.int32)
    tw = np.random.default_rng(k + 1).uniform(0.1, 1.0, 9).astype(np.float32)
    got = moe_into(stack, xs, k, sorted_ids, expert_ids, tw, topk, 9)
    check_against_forward(stack, xs, got, sorted_ids, expert_ids, tw, topk)
    sel = [0, 6, 8]
    check_against_oracle(qtype, stack, x, got, sorted_ids[sel], expert_ids[sel], tw, topk)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("k", [256, 768, 1280, 2048])
def test_moe_kquant_short_rows_packed(name, k):
    """Rows of at most 8 super-blocks run 2 or 4 rows a wave; an expert of
    37 rows leaves a partial pack. Each pair still equals its own
    qmm_forward bit for bit, and the oracle."""
    qtype = MOE_TYPES[name]
    E, n, tokens, topk = 5, 37, 7, 3
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, k + 5)
    stack = expert_stack(qtype, E, n, k, k + 7)
    x = np.random.default_rng(k).standard_normal((tokens * topk, k)).astype(np.float32)
    xs = t32(x)
    got = moe_into(stack, xs, k, sorted_ids, expert_ids, topk_w, topk, tokens * topk)
    assert not np.isnan(got).any()
    check_against_forward(stack, xs, got, sorted_ids, expert_ids, topk_w, topk)
    check_against_oracle(qtype, stack, x, got, sorted_ids, expert_ids, topk_w, topk)
