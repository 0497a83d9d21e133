"""Prompt grouped expert products (qmm_moe_forward_prefill, the reference's
moe_gemm_gguf_prefill) against the CPU oracle, through the C ABI, for every
type and input type (f16, bf16, f32 rounded to f16).

The weights each product uses are the to_float values rounded to the 16-bit
type bit for bit (one-hot input rows return them exactly); the sums are
checked against the oracle's f64 sum of the same rounded operands, within
the north star's 2e-3 GEMM bound normalised by ||w|| ||x|| (the observed
error is that of an f32 sum, about 1e-6). Routing as tests/test_moe_gpu.py
draws it.
"""
import ctypes
import zlib

import numpy as np
import pytest
import torch

from helpers import TOL_GEMM, normalised_error
from oracle import qref
from swarmllm_amd import QTensor, moe_forward, moe_uses_prompt_kernel
from swarmllm_amd._lib import QMM_UNSUPPORTED, QMM_WORKSPACE_TOO_SMALL, X_BF16, X_F16, X_F32, lib
from test_moe_gpu import MOE_TYPES, expert_stack, routing, t32

pytestmark = pytest.mark.gpu

DEV = "cuda"
KQUANT = {12, 14}
TORCH_X = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def check_prefill(qtype, stack, x, out, sorted_ids, expert_ids, topk_w, topk, bf16):
    """Each listed entry's output row against the oracle (a sample of a
    routing's entries may be listed: out holds all of its rows)."""
    e, n, k = stack.shape
    wb = stack.data_.cpu().numpy()
    want = qref.moe_prefill(qtype, wb, e, n, k, x, bf16, sorted_ids, expert_ids, topk_w, topk, out.shape[0])
    rnd = qref.round_bf16 if bf16 else qref.round_f16
    per = wb.size // e
    worst = 0.0
    for i in range(len(sorted_ids)):
        p, ex = int(sorted_ids[i]), int(expert_ids[i])
        row = p if topk_w is not None else p // topk
        scale = np.float32(topk_w[p]) if topk_w is not None else np.float32(1.0)
        wdeq = rnd(qref.to_float(qtype, wb[ex * per:(ex + 1) * per], n * k).reshape(n, k))
        err = normalised_error(out[p][None, :], want[p][None, :], wdeq, (rnd(x[row]) * scale)[None, :])
        worst = max(worst, err)
    assert worst <= TOL_GEMM, f"worst normalised error {worst}"
    return worst


@pytest.mark.parametrize("name", list(MOE_TYPES))
@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
def test_prefill_one_hot_rows_return_rounded_weights(name, xdt):
    """Input rows e_c: each output is the weight column c rounded to the 16-bit
    type, bit for bit, for every weight row, including a partial last tile."""
    qtype = MOE_TYPES[name]
    E, n, topk, tokens = 4, 300, 2, 24
    k = 512 if qtype in KQUANT else 352
    seed = zlib.crc32(f"onehot-{name}-{xdt}".encode())
    sorted_ids, expert_ids, _ = routing(tokens, E, topk, seed)
    stack = expert_stack(qtype, E, n, k, seed & 0xFFFF)
    cols = np.random.default_rng(seed).integers(0, k, tokens)
    x = np.zeros((tokens, k), np.float32)
    x[np.arange(tokens), cols] = 1.0
    xs = torch.from_numpy(x).to(DEV).to(TORCH_X[xdt])
    out = moe_forward(xs, stack, t32(sorted_ids), t32(expert_ids), None, topk, prompt=True).cpu().numpy()
    rnd = qref.round_bf16 if xdt == "bf16" else qref.round_f16
    wb = stack.data_.cpu().numpy()
    per = wb.size // E
    for p, ex in zip(sorted_ids, expert_ids):
        w = qref.to_float(qtype, wb[ex * per:(ex + 1) * per], n * k).reshape(n, k)
        want = rnd(w[:, cols[p // topk]]) + np.float32(0.0)
        assert np.array_equal(out[p].view(np.uint32), want.view(np.uint32)), f"pair {p} expert {ex}"


@pytest.mark.parametrize("name", list(MOE_TYPES))
@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("weighted", [False, True])
def test_prefill_parity(name, xdt, weighted):
    """40 tokens top-3 over 8 experts: runs longer than a 32-entry chunk, a
    partial weight tile (n = 300) and, for the 32-value formats, a partial
    last stage (k = 352)."""
    qtype = MOE_TYPES[name]
    E, n, tokens, topk = 8, 300, 40, 3
    k = 768 if qtype in KQUANT else 352
    seed = zlib.crc32(f"pf-{name}-{xdt}-{weighted}".encode())
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, seed)
    stack = expert_stack(qtype, E, n, k, seed & 0xFFFF)
    rows = tokens * topk if weighted else tokens
    x = np.random.default_rng(seed).standard_normal((rows, k)).astype(np.float32)
    xs = torch.from_numpy(x).to(DEV).to(TORCH_X[xdt])
    xr = xs.float().cpu().numpy()  # the 16-bit input as the kernel reads it (f32: rounded in the library)
    tw = topk_w if weighted else None
    before = lib().qmm_moe_prefill_launches()
    out = moe_forward(xs, stack, t32(sorted_ids), t32(expert_ids), t32(topk_w) if weighted else None, topk,
                      prompt=True).cpu().numpy()
    assert lib().qmm_moe_prefill_launches() == before + 1
    check_prefill(qtype, stack, xr, out, sorted_ids, expert_ids, tw, topk, xdt == "bf16")


def prefill_into(stack, xs, x_dtype, x_stride, sorted_ids, expert_ids, topk_w, topk, rows_out,
                 fill=float("nan")):
    """qmm_moe_forward_prefill through the C ABI into an output prefilled with `fill`."""
    L = lib()
    e, n, k = stack.shape
    out = torch.full((rows_out, n), fill, dtype=torch.float32, device=DEV)
    size_m = len(sorted_ids)
    sid, eid = t32(sorted_ids), t32(expert_ids)
    tw = t32(topk_w) if topk_w is not None else None
    need = ctypes.c_size_t(0)
    args = (int(stack.dtype), stack.data_.data_ptr(), e, xs.data_ptr(), x_dtype, x_stride, sid.data_ptr(),
            eid.data_ptr(), tw.data_ptr() if tw is not None else None, topk, out.data_ptr(), n)
    assert L.qmm_moe_forward_prefill(*args, None, 0, ctypes.byref(need), k, n, size_m, 0, 0) == 0
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    assert L.qmm_moe_forward_prefill(*args, ws.data_ptr(), ws.numel(), ctypes.byref(need), k, n, size_m, 1, 0) == 0
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("name", ["Q4_K", "MXFP4"])
def test_prefill_strided_and_unaligned_inputs_match_contiguous(name):
    """Input rows x_stride apart (a stride that is not a multiple of 8 values
    is copied aligned first) give the contiguous input's results bit for bit."""
    qtype = MOE_TYPES[name]
    E, n, tokens, topk = 6, 96, 20, 2
    k = 512 if qtype in KQUANT else 320
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, 91)
    stack = expert_stack(qtype, E, n, k, 92)
    x = np.random.default_rng(93).standard_normal((tokens, k)).astype(np.float32)
    base = prefill_into(stack, t32(x).half(), X_F16, k, sorted_ids, expert_ids, None, topk, tokens * topk)
    for extra in (8, 3):
        padded = np.zeros((tokens, k + extra), np.float32)
        padded[:, :k] = x
        got = prefill_into(stack, t32(padded).half(), X_F16, k + extra, sorted_ids, expert_ids, None, topk,
                           tokens * topk)
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), f"stride {k + extra}"
    got = prefill_into(stack, t32(x), X_F32, k, sorted_ids, expert_ids, None, topk, tokens * topk)
    assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), "f32 input rounded to f16"


def test_prefill_order_of_entries_and_out_of_range_entries():
    qtype = MOE_TYPES["Q6_K"]
    E, n, k, tokens, topk = 6, 128, 512, 30, 2
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, 17)
    stack = expert_stack(qtype, E, n, k, 18)
    x = np.random.default_rng(19).standard_normal((tokens * topk, k)).astype(np.float32)
    xs = t32(x).half()
    ref = prefill_into(stack, xs, X_F16, k, sorted_ids, expert_ids, topk_w, topk, tokens * topk)
    check_prefill(qtype, stack, xs.float().cpu().numpy(), ref, sorted_ids, expert_ids, topk_w, topk, False)
    # entries in any order: the same sums (each within its own chunk position)
    perm = np.random.default_rng(20).permutation(len(sorted_ids))
    got = prefill_into(stack, xs, X_F16, k, sorted_ids[perm], expert_ids[perm], topk_w, topk, tokens * topk)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    # an out-of-range expert or pair writes nothing
    eid = expert_ids.copy()
    sid = sorted_ids.copy()
    eid[0] = E
    eid[5] = -1
    sid[9] = tokens * topk + 4
    got = prefill_into(stack, xs, X_F16, k, sid, eid, topk_w, topk, tokens * topk + 8)
    skipped = {int(sorted_ids[0]), int(sorted_ids[5]), int(sorted_ids[9])}
    for p in range(tokens * topk + 8):
        if p in skipped or p >= tokens * topk:
            assert np.isnan(got[p]).all(), f"row {p} was written"
        else:
            assert np.array_equal(got[p].view(np.uint32), ref[p].view(np.uint32)), f"row {p}"


def test_prefill_qwen3_moe_like_and_gpt_oss_shapes():
    """128 experts of a 2048-wide MoE layer (expert width 768, top-8), gate+up
    Q4_K [1536, 2048] and down Q6_K [2048, 768], 64 tokens; and BASELINE C4's
    gpt-oss-20b experts (MXFP4, 32 x [5760, 2880] and [2880, 2880], top-4),
    64 tokens. Oracle-checked on a sample of entries."""
    for qg, qd, E, hidden, inter, topk, tokens, seed in [(12, 14, 128, 2048, 768, 8, 64, 41),
                                                         (39, 39, 32, 2880, 2880, 4, 64, 42)]:
        assert moe_uses_prompt_kernel(tokens)
        sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, seed)
        gate = expert_stack(qg, E, 2 * inter, hidden, seed)
        down = expert_stack(qd, E, hidden, inter, seed + 1)
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((tokens, hidden)).astype(np.float32)
        y1 = moe_forward(t32(x), gate, t32(sorted_ids), t32(expert_ids), None, topk, prompt=True).cpu().numpy()
        x2 = rng.standard_normal((tokens * topk, inter)).astype(np.float32)
        y2 = moe_forward(t32(x2), down, t32(sorted_ids), t32(expert_ids), t32(topk_w), topk,
                         prompt=True).cpu().numpy()
        pick = rng.choice(len(sorted_ids), 24, replace=False)
        check_prefill(qg, gate, x, y1, sorted_ids[pick], expert_ids[pick], None, topk, False)
        check_prefill(qd, down, x2, y2, sorted_ids[pick], expert_ids[pick], topk_w, topk, False)


def test_prefill_status_paths():
    L = lib()
    need = ctypes.c_size_t(0)
    # Q4_K rows must hold whole super-blocks
    assert L.qmm_moe_forward_prefill(12, None, 4, None, X_F16, 320, None, None, None, 2, None, 64, None, 0,
                                     ctypes.byref(need), 320, 64, 8, 0, 0) == QMM_UNSUPPORTED
    # an unknown input type
    assert L.qmm_moe_forward_prefill(39, None, 4, None, 7, 320, None, None, None, 2, None, 64, None, 0,
                                     ctypes.byref(need), 320, 64, 8, 0, 0) == QMM_UNSUPPORTED
    assert L.qmm_moe_forward_prefill(39, None, 4, None, X_BF16, 320, None, None, None, 2, None, 64, None, 0,
                                     ctypes.byref(need), 320, 64, 8, 0, 0) == 0 and need.value > 0
    stack = expert_stack(39, 4, 64, 320, 5)
    x = torch.zeros((4, 320), dtype=torch.bfloat16, device=DEV)
    sid, eid = t32(np.arange(8, dtype=np.int32)), t32(np.repeat(np.arange(4, dtype=np.int32), 2))
    out = torch.empty((8, 64), dtype=torch.float32, device=DEV)
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    assert L.qmm_moe_forward_prefill(39, stack.data_.data_ptr(), 4, x.data_ptr(), X_BF16, 320, sid.data_ptr(),
                                     eid.data_ptr(), None, 2, out.data_ptr(), 64, ws.data_ptr(), need.value - 1,
                                     ctypes.byref(need), 320, 64, 8, 1, 0) == QMM_WORKSPACE_TOO_SMALL
    assert L.qmm_moe_forward_prefill(39, stack.data_.data_ptr(), 4, x.data_ptr(), X_BF16, 320, sid.data_ptr(),
                                     eid.data_ptr(), None, 2, out.data_ptr(), 64, ws.data_ptr(), ws.numel(),
                                     ctypes.byref(need), 320, 64, 8, 1, 0) == 0
    torch.cuda.synchronize()
    assert (out == 0).all()
    assert X_F16 == 0 and X_F32 == 2


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "MXFP4", "Q8_0"])
def test_prefill_runs_longer_than_a_chunk(name):
    """Two experts each chosen by all 100 tokens (runs of 100 entries: a
    64-entry chunk and a 36-entry one) and a third expert chosen by 32 tokens
    (exactly one row tile), per-pair inputs and routing weights."""
    qtype = MOE_TYPES[name]
    E, n, topk = 3, 160, 2
    k = 512 if qtype in KQUANT else 384
    tokens = 100
    pairs = []
    for t in range(tokens):
        second = 2 if t < 32 else 1
        pairs += [(0, t * topk), (second, t * topk + 1)]
    pairs.sort()
    expert_ids = np.array([e for e, _ in pairs], np.int32)
    sorted_ids = np.array([p for _, p in pairs], np.int32)
    rng = np.random.default_rng(123)
    topk_w = rng.random(tokens * topk).astype(np.float32)
    stack = expert_stack(qtype, E, n, k, 124)
    x = rng.standard_normal((tokens * topk, k)).astype(np.float32)
    xs = t32(x).half()
    out = prefill_into(stack, xs, X_F16, k, sorted_ids, expert_ids, topk_w, topk, tokens * topk)
    check_prefill(qtype, stack, xs.float().cpu().numpy(), out, sorted_ids, expert_ids, topk_w, topk, False)


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_prefill_mxfp4_every_code_at_extreme_scales(xdt):
    """MXFP4 blocks with every E2M1 code under scale bytes 0, 1, 2, 100-160,
    200, 254 and 255 (subnormal, overflowing and NaN-coded scales), read back
    through one-hot input rows: each output equals the oracle's, bit for bit
    (NaN where a zero input meets an infinite weight, in both)."""
    from swarmllm_amd import GgmlDType

    n, k = 32, 64
    scales = [0, 1, 2, 254, 255] + list(range(100, 161, 3)) + [200]
    rng = np.random.default_rng(5)
    blocks = []
    for j in range(n):
        for b in range(k // 32):
            e = scales[(2 * j + b) % len(scales)]
            qs = rng.integers(0, 256, 16, dtype=np.uint8)
            qs[:8] = np.arange(16, dtype=np.uint8)[::2] | (np.arange(16, dtype=np.uint8)[1::2] << 4)
            blocks.append(np.concatenate([[e], qs]).astype(np.uint8))
    wb = np.concatenate(blocks)
    stack = QTensor(torch.from_numpy(wb).to(DEV), (1, n, k), GgmlDType(39))
    x = np.eye(k, dtype=np.float32)
    sorted_ids = np.arange(k, dtype=np.int32)
    expert_ids = np.zeros(k, np.int32)
    xs = torch.from_numpy(x).to(DEV).to(TORCH_X[xdt])
    out = prefill_into(stack, xs, X_BF16 if xdt == "bf16" else X_F16, k, sorted_ids, expert_ids, None, 1, k)
    want = qref.moe_prefill(39, wb, 1, n, k, x, xdt == "bf16", sorted_ids, expert_ids, None, 1)
    assert np.array_equal(np.isnan(out), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal((out[fin] + np.float32(0)).view(np.uint32), (want[fin] + np.float32(0)).view(np.uint32))
