"""The rest of the device arm's surface (QCudaStorage, quantized/
dummy_cuda.rs:10-143) as the reference's callers use it:
  - gather_rows: the quantized embedding lookup (mod.rs:1039-1091,
    cuda.rs:1478-1540), checked against byte slicing of the table;
  - quantize_onto (mod.rs:907-932) and accumulate_in_f32 (mod.rs:1181-1200);
  - indexed_moe_forward's [batch, topk] layout (mod.rs:1093-1118,
    cuda.rs:1236-1376) served by qmm_moe_forward;
  - the loader variants: load_quantized_entries / _beside, chosen entries
    of a stack from the file, pinned_load_chunks and the SWARMLLM_LOAD_PINNED
    / SWARMLLM_LOAD_READ switches (cuda.rs:1966-2127, gguf_file.rs:57-63);
  - qmm_prepare: a product whose first call is under a graph capture
    (mmq_prepare_few_rows_once, cuda.rs:890-932).
"""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest
import torch

from golden import make_tiny_gguf as tiny
from helpers import TOL_GEMM, TOL_MATVEC, normalised_error
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal
from swarmllm_amd._lib import QMM_OK, QMM_UNSUPPORTED, QmmError, lib
from swarmllm_amd.gguf import (Content, load_quantized_beside, load_quantized_entries, pinned_load_chunks,
                               with_pinned_load_staging)

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
V3 = f"{tiny.HERE}/tiny_v3.gguf"

FORMATS = [GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q6K, GgmlDType.Iq4Nl, GgmlDType.Mxfp4]


def table(dtype, vocab, hidden, seed):
    return QTensor.quantize(fill_normal(vocab * hidden, seed=seed, std=0.5).reshape(vocab, hidden), dtype)


# hidden sizes whose rows take each copy width: 16-byte units (Q4_K 2 blocks,
# Q8_0 8 blocks = 272 B), 4-byte units (Q8_0 2 blocks = 68 B), bytes (MXFP4 3
# blocks = 51 B, IQ4_NL 1 block = 18 B)
CASES = [(GgmlDType.Q4K, 512), (GgmlDType.Q6K, 768), (GgmlDType.Q8_0, 256), (GgmlDType.Q8_0, 64),
         (GgmlDType.Mxfp4, 96), (GgmlDType.Iq4Nl, 32), (GgmlDType.Mxfp4, 2880)]


@pytest.mark.parametrize("dtype,hidden", CASES, ids=[f"{d.name}-{h}" for d, h in CASES])
def test_gather_rows_equals_byte_slicing(dtype, hidden):
    vocab = 300
    t = table(dtype, vocab, hidden, seed=hidden + int(dtype))
    ids_host = np.array([0, 299, 7, 7, 123, 1, 298, 42, 0], np.int64)
    ids = torch.from_numpy(ids_host).to(torch.uint32).cuda()
    g = t.gather_rows(ids)
    assert g.shape == (len(ids_host), hidden) and g.dtype == dtype
    rb = hidden // dtype.block_size() * dtype.type_size()
    raw = np.frombuffer(t.data(), np.uint8).reshape(vocab, rb)
    assert g.data() == raw[ids_host].tobytes()
    # padded as a device weight, the padding zero
    assert g.padded_bytes() == lib().qmm_padded_bytes(int(dtype), len(ids_host) * hidden)
    assert int(g.storage_[g.data_.numel():].abs().sum().item()) == 0
    # the rows dequantize to the table's rows
    assert torch.equal(g.dequantize(), t.dequantize()[torch.from_numpy(ids_host).cuda()])


def test_gather_rows_edges():
    t = table(GgmlDType.Q4K, 50, 256, seed=3)
    raw = np.frombuffer(t.data(), np.uint8).reshape(50, 144)
    # 0xFFFFFFFF: index_select's "no row", a zero row
    g = t.gather_rows(torch.tensor([4, 0xFFFFFFFF, 49], dtype=torch.int64).to(torch.uint32).cuda())
    got = np.frombuffer(g.data(), np.uint8).reshape(3, 144)
    assert np.array_equal(got[0], raw[4]) and np.array_equal(got[2], raw[49]) and not got[1].any()
    assert not g.dequantize()[1].abs().sum().item()
    # an id past the vocabulary is refused, as the host path refuses it
    with pytest.raises(ValueError, match="id 50 out of range for vocabulary 50"):
        t.gather_rows(torch.tensor([1, 50, 2], dtype=torch.int64).to(torch.uint32).cuda())
    # without the check (no readback) that row is zero
    g = t.gather_rows(torch.tensor([1, 1000], dtype=torch.int64).to(torch.uint32).cuda(), check_ids=False)
    got = np.frombuffer(g.data(), np.uint8).reshape(2, 144)
    assert np.array_equal(got[0], raw[1]) and not got[1].any()
    # the device counter: one per refused id
    L = lib()
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty(4 * 144, dtype=torch.uint8, device="cuda")
    ids = torch.tensor([60, 2, 0xFFFFFFFF, 51], dtype=torch.int64).to(torch.uint32).cuda()
    assert L.qmm_gather_rows(12, t.data_.data_ptr(), t.data_.numel(), 50, 256, ids.data_ptr(), 4, out.data_ptr(),
                             out.numel(), bad.data_ptr(), torch.cuda.current_stream().cuda_stream) == QMM_OK
    torch.cuda.synchronize()
    assert int(bad.item()) == 2
    # empty ids; u32 required; 2-D required; whole blocks; a table too small
    assert t.gather_rows(torch.zeros(0, dtype=torch.int64).to(torch.uint32).cuda()).shape == (0, 256)
    with pytest.raises(ValueError, match="u32"):
        t.gather_rows(torch.tensor([1], dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError, match="2-D"):
        QTensor.alloc((2, 3, 256), GgmlDType.Q4K).gather_rows(torch.zeros(1, dtype=torch.int64).to(torch.uint32).cuda())
    assert L.qmm_gather_rows(12, t.data_.data_ptr(), t.data_.numel(), 50, 200, ids.data_ptr(), 4, out.data_ptr(),
                             out.numel(), None, 0) == QMM_UNSUPPORTED
    assert L.qmm_gather_rows(12, t.data_.data_ptr(), 49 * 144, 50, 256, ids.data_ptr(), 4, out.data_ptr(),
                             out.numel(), None, 0) == QMM_UNSUPPORTED


def test_gather_rows_then_dequantize_f16_is_the_embedding_lookup():
    """The caller's use (src/inference/split/token_embedding.rs:225-255):
    gather the token rows, dequantize_f16, reshape to [*ids, hidden]."""
    t = table(GgmlDType.Q8_0, 1000, 2048, seed=11)
    ids = torch.tensor([[5, 999], [0, 5]], dtype=torch.int64)
    rows = t.gather_rows(ids.reshape(-1).to(torch.uint32).cuda())
    emb = rows.dequantize_f16().reshape(2, 2, 2048)
    want = t.dequantize_f16()[ids.reshape(-1).cuda()].reshape(2, 2, 2048)
    assert torch.equal(emb, want)


def test_quantize_onto_matches_quantize():
    rng = np.random.default_rng(4)
    for dtype in FORMATS:
        src = torch.from_numpy(rng.standard_normal((3, 8, 512)).astype(np.float32))
        q = QTensor.quantize_onto(src, dtype)
        assert q.shape == (3, 8, 512)
        assert q.data() == QTensor.quantize(src.reshape(24, 512).cuda(), dtype).data()
    with pytest.raises(ValueError, match="cpu"):
        QTensor.quantize_onto(torch.zeros((2, 256), device="cuda"), GgmlDType.Q4K)
    with pytest.raises(ValueError, match="divisible"):
        QTensor.quantize_onto(torch.zeros((2, 100)), GgmlDType.Q8_0)


def test_accumulate_in_f32_changes_nothing():
    mm = QMatMul(table(GgmlDType.Q4K, 1024, 2048, seed=12))
    for rows in (1, 5, 200):
        x = fill_normal(rows * 2048, seed=rows).reshape(rows, 2048)
        before = mm.forward(x)
        assert mm.accumulate_in_f32() is True
        assert torch.equal(mm.forward(x), before)
    assert lib().qmm_accumulate_in_f32(3) == QMM_UNSUPPORTED


MOE = [(GgmlDType.Q4K, 256, 512), (GgmlDType.Q6K, 128, 512), (GgmlDType.Q8_0, 192, 256), (GgmlDType.Mxfp4, 96, 288)]


@pytest.mark.parametrize("dtype,n,k", MOE, ids=[d.name for d, _, _ in MOE])
@pytest.mark.parametrize("shared", [True, False], ids=["x_b1k", "x_btk"])
def test_indexed_moe_forward_layout(dtype, n, k, shared):
    """ids [batch, topk] unsorted (repeats included), x [batch, 1|topk, k]:
    out[b, j] is the product of x[b, 0|j] with expert ids[b, j], each equal
    bit for bit to that expert's own QMatMul.forward, and within the oracle's
    tolerance."""
    E, batch, topk = 6, 5, 3
    w = QTensor.quantize(fill_normal(E * n * k, seed=int(dtype) * 7 + n, std=0.02).reshape(E * n, k), dtype)
    stack = QTensor(w.storage_, (E, n, k), dtype)
    ids_host = np.array([[5, 0, 2], [2, 2, 1], [0, 4, 5], [3, 1, 0], [4, 5, 3]], np.int64)
    ids = torch.from_numpy(ids_host).to(torch.uint32).cuda()
    x = fill_normal(batch * (1 if shared else topk) * k, seed=k + n).reshape(batch, 1 if shared else topk, k)
    y = QMatMul(stack).indexed_moe_forward(x, ids)
    assert y.shape == (batch, topk, n)
    per = w.data_.numel() // E
    raw = np.frombuffer(w.data(), np.uint8)
    xh = x.cpu().numpy()
    for b in range(batch):
        for j in range(topk):
            e = int(ids_host[b, j])
            xe = x[b, 0 if shared else j].reshape(1, k).contiguous()
            expert = QTensor(w.data_[e * per:(e + 1) * per].clone(), (n, k), dtype)
            assert torch.equal(y[b, j], QMatMul(expert).forward(xe)[0]), (b, j)
    # the oracle on one token's slots
    eraw = raw[int(ids_host[1, 2]) * per:(int(ids_host[1, 2]) + 1) * per]
    xr = xh[1, 0 if shared else 2].reshape(1, k)
    want = qref.matmul(int(dtype), xr, eraw, n)
    wdeq = qref.to_float(int(dtype), eraw, n * k).reshape(n, k)
    assert normalised_error(y[1, 2].cpu().numpy().reshape(1, n), want, wdeq, xr) <= TOL_MATVEC
    # an expert id out of range leaves its slot zero
    ids_bad = ids.clone()
    ids_bad[0, 1] = E + 3
    yb = QMatMul(stack).indexed_moe_forward(x, ids_bad)
    assert not yb[0, 1].abs().sum().item()
    assert torch.equal(yb[0, 0], y[0, 0]) and torch.equal(yb[2], y[2])


def test_load_quantized_entries_and_beside():
    c = Content.read(V3)
    stack = c.tensor("blk.0.ffn_gate_exps.weight")  # [4, 32, 64] MXFP4
    e, n, k = stack.shape
    per = stack.data_.numel() // e
    raw = stack.data()
    parts = [(0, raw[3 * per:4 * per]), (4, raw[1 * per:2 * per])]
    q = load_quantized_entries(stack.dtype, 5, (n, k), parts)
    assert q.shape == (5, n, k) and q.padded_bytes() == lib().qmm_padded_bytes(int(stack.dtype), 5 * n * k)
    got = q.storage_.cpu().numpy()
    assert got[:per].tobytes() == raw[3 * per:4 * per] and got[4 * per:5 * per].tobytes() == raw[per:2 * per]
    assert not got[per:4 * per].any() and not got[5 * per:].any()
    with pytest.raises(ValueError, match="slot 5 of 5"):
        load_quantized_entries(stack.dtype, 5, (n, k), [(5, raw[:per])])
    with pytest.raises(ValueError, match="expected"):
        load_quantized_entries(stack.dtype, 5, (n, k), [(1, raw[:per - 17])])
    # beside: a side stream's copy, the current stream waits for it
    w = c.tensor("blk.0.ffn_down.weight")
    b = load_quantized_beside(w.data(), w.shape, w.dtype)
    x = torch.from_numpy(np.random.default_rng(2).standard_normal((3, w.shape[1])).astype(np.float32)).cuda()
    assert b.data() == w.data() and int(b.storage_[b.data_.numel():].abs().sum().item()) == 0
    assert torch.equal(QMatMul(b).forward(x), QMatMul(w).forward(x))
    assert with_pinned_load_staging(lambda: 7) == 7


def test_stack_entries_from_the_file():
    c = Content.read(V3)
    full = c.tensor("blk.0.ffn_gate_exps.weight")
    e = full.shape[0]
    per = full.data_.numel() // e
    q = c.tensor_entries("blk.0.ffn_gate_exps.weight", [2, 0, 2])
    assert q.shape == full.shape and q.padded_bytes() == full.padded_bytes()
    got, want = q.storage_.cpu().numpy(), full.storage_.cpu().numpy()
    for s in range(e):
        span = slice(s * per, (s + 1) * per)
        if s in (0, 2):
            assert np.array_equal(got[span], want[span]), s
        else:
            assert not got[span].any(), s
    assert not got[e * per:].any()
    with pytest.raises(ValueError, match="slot 4 of 4"):
        c.tensor_entries("blk.0.ffn_gate_exps.weight", [4])
    with pytest.raises(ValueError, match="not a stack"):
        c.tensor_entries("rope_freqs", [0])


def big_file(path, n=2048, k=19456, truncate=0):
    """A GGUF of one Q8_0 tensor of 42 MB (three 16 MiB staging chunks) of
    random bytes; `truncate` drops that many bytes off the end."""
    nbytes = n * (k // 32) * 34
    data = np.random.default_rng(7).integers(0, 256, nbytes, dtype=np.uint8)
    pre = struct.pack("<II", 0x46554747, 3) + struct.pack("<QQ", 1, 0)
    pre += tiny._str("big", 3) + struct.pack("<I", 2) + struct.pack("<QQ", k, n) + struct.pack("<IQ", 8, 0)
    pre += b"\x00" * ((-len(pre)) % 32)
    path.write_bytes((pre + data.tobytes())[:len(pre) + nbytes - truncate])
    return data


def test_pinned_chunks_and_a_truncated_file(tmp_path):
    p = tmp_path / "big.gguf"
    data = big_file(p)
    c0 = pinned_load_chunks()
    q = Content.read(str(p)).tensor("big")
    assert np.array_equal(q.data_.cpu().numpy(), data)
    assert pinned_load_chunks() - c0 == 3
    # a tensor running past the file's end is refused before any copy
    t = tmp_path / "cut.gguf"
    big_file(t, truncate=1000)
    c = Content.read(str(t))
    q = QTensor.alloc((2048, 19456), GgmlDType.Q8_0)
    q.storage_.fill_(0xAB)
    st = lib().qmm_gguf_load(c._h, c.tensor_infos["big"].index, q.storage_.data_ptr(), q.storage_.numel(),
                             torch.cuda.current_stream().cuda_stream)
    assert st == QMM_UNSUPPORTED
    torch.cuda.synchronize()
    assert int((q.storage_ != 0xAB).sum().item()) == 0
    with pytest.raises(QmmError):
        c.tensor("big")


def run_child(args, env=None, timeout=300):
    """fresh_child.py in a process of its own (the package on its path), its
    switches set: a process reads them once."""
    full = {k: v for k, v in os.environ.items() if not k.startswith("SWARMLLM_LOAD")}
    full.update(env or {})
    full["PYTHONPATH"] = ROOT + (os.pathsep + full["PYTHONPATH"] if full.get("PYTHONPATH") else "")
    print(f"child {args[0]} with {env}", flush=True)
    res = subprocess.run([sys.executable, "-u", os.path.join(HERE, "fresh_child.py"), *args], env=full, cwd=ROOT,
                         capture_output=True, text=True, timeout=timeout)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]


@pytest.mark.parametrize("env", [{"SWARMLLM_LOAD_PINNED": "0"}, {"SWARMLLM_LOAD_READ": "fresh"}],
                         ids=["pinned_off", "read_fresh"])
def test_loader_switches(tmp_path, env):
    """The switches move the copy off the pinned pair; the bytes arrive whole."""
    p = tmp_path / "big.gguf"
    data = big_file(p)
    out = str(tmp_path / "o.npz")
    run_child(["load", str(p), "big", out], env)
    r = np.load(out)
    assert np.array_equal(r["data"], data) and not r["pad"].any()
    assert int(r["chunks"][0]) == 0


def test_first_product_under_capture(tmp_path):
    """In a fresh process: a 4-row Q4_K product captured before anything
    prepared its type runs on the decode kernels (the reference lets a
    captured few-rows product take the matrix cores only once prepared);
    the same product outside a capture prepares Q4_K and takes the few-row
    matrix-core kernel, which a second capture then takes too, its replays
    equal to the eager call bit for bit. A GEMM whose kernel first runs under
    capture and the no-allocation entry's first call under capture (after
    qmm_prepare) replay to the eager results bit for bit."""
    out = str(tmp_path / "c.npz")
    run_child(["capture", out])
    r = np.load(out)
    assert not r["prepared_before"][0] and not r["prepared_after_capture"][0] and r["prepared_after_eager"][0]
    # launch_sk: the few-row matrix-core kernel's launcher
    assert "launch_sk" not in str(r["kernel_first"]), str(r["kernel_first"])
    assert "launch_sk" in str(r["kernel_eager"]) and "launch_sk" in str(r["kernel_second"])
    assert np.array_equal(r["y_second0"], r["y_eager"]) and np.array_equal(r["y_second1"], r["y_eager"])
    # the first (decode-kernel) product against the oracle
    w = QTensor.quantize(fill_normal(4096 * 4096, seed=91, std=0.02).reshape(4096, 4096), GgmlDType.Q4K)
    x = fill_normal(4 * 4096, seed=92).reshape(4, 4096).cpu().numpy()
    raw = np.frombuffer(w.data(), np.uint8)
    want = qref.matmul(12, x, raw, 4096)
    wdeq = qref.to_float(12, raw, 4096 * 4096).reshape(4096, 4096)
    assert normalised_error(r["y_first"], want, wdeq, x) <= TOL_MATVEC
    assert normalised_error(r["y_eager"], want, wdeq, x) <= TOL_GEMM
    assert "gemm" in str(r["kernel_gemm"])
    assert np.array_equal(r["y_gemm_captured"], r["y_gemm_eager"])
    assert int(r["noalloc_status"][0]) == QMM_OK
    assert np.array_equal(r["y_noalloc_captured"], r["y_noalloc_eager"])
