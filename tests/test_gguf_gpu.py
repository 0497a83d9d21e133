"""GGUF tensors into device QTensors (qmm_gguf_load: Content::tensor ->
ggml_file::qtensor_read -> cuda::load_quantized_read, gguf_file.rs:489-500,
ggml_file.rs:220-256, cuda.rs:1846-2075): bytes identical to the file's,
512 values' worth of zeroed padding past them (MATRIX_ROW_PADDING), products
on the loaded weights equal to products on the same bytes uploaded directly
and within the tolerance of the CPU oracle; expert stacks (stack_some)."""
import struct

import numpy as np
import pytest
import torch

from golden import make_tiny_gguf as tiny
from helpers import TOL_MATVEC, normalised_error
from oracle import qref
from swarmllm_amd import GgmlDType, QMatMul, QTensor, moe_forward
from swarmllm_amd._lib import lib
from swarmllm_amd.gguf import Content

pytestmark = pytest.mark.gpu

V3 = f"{tiny.HERE}/tiny_v3.gguf"


def file_bytes(path, c, name):
    info = c.tensor_infos[name]
    with open(path, "rb") as f:
        f.seek(c.tensor_data_offset + info.offset)
        return f.read(info.nbytes)


@pytest.mark.parametrize("name", [t[0] for t in tiny.TENSORS_V3])
def test_load_round_trips_the_files_bytes_with_zero_padding(name):
    c = Content.read(V3)
    q = c.tensor(name)
    raw = file_bytes(V3, c, name)
    assert q.data() == raw  # QTensor::data round trip
    assert q.shape == c.tensor_infos[name].shape
    n = int(np.prod(q.shape))
    assert q.padded_bytes() == lib().qmm_padded_bytes(int(q.dtype), n) > len(raw)
    assert int(q.storage_[len(raw):].abs().sum().item()) == 0


def test_loaded_weights_multiply_like_uploaded_bytes_and_the_oracle():
    c = Content.read(V3)
    rng = np.random.default_rng(5)
    for name, t, shape in tiny.TENSORS_V3:
        if len(shape) != 2 or t not in (8, 12, 14, 20, 39):
            continue
        q = c.tensor(name)
        raw = np.frombuffer(file_bytes(V3, c, name), np.uint8)
        n, k = shape
        x = rng.standard_normal((3, k)).astype(np.float32)
        xt = torch.from_numpy(x).cuda()
        y = QMatMul(q).forward(xt)
        assert torch.equal(y, QMatMul(QTensor.from_data(raw.tobytes(), shape, GgmlDType(t))).forward(xt))
        want = qref.matmul(t, x, raw, n)
        wdeq = qref.to_float(t, raw, n * k).reshape(n, k)
        assert normalised_error(y.cpu().numpy(), want, wdeq, x) <= TOL_MATVEC, name


def test_f32_and_f16_tensors_hold_their_values():
    c = Content.read(V3)
    norm = c.tensor("output_norm.weight").dequantize().cpu().numpy()
    assert np.array_equal(norm, np.frombuffer(file_bytes(V3, c, "output_norm.weight"), "<f4"))
    rope = c.tensor("rope_freqs").dequantize().cpu().numpy()
    assert np.array_equal(rope, np.frombuffer(file_bytes(V3, c, "rope_freqs"), "<f2").astype(np.float32))
    with pytest.raises(Exception):
        QMatMul(c.tensor("output_norm.weight")).forward(torch.zeros((1, 96), device="cuda"))


def test_load_across_staging_chunks(tmp_path):
    """A tensor of 42 MB crosses the 16 MiB staging chunks; its bytes (random:
    only the copy is checked) arrive whole."""
    n, k = 2048, 19456
    nbytes = n * (k // 32) * 34
    data = np.random.default_rng(7).integers(0, 256, nbytes, dtype=np.uint8)
    # magic, version 3, one tensor, one key/value; the tensor's info; padding to 32
    pre = struct.pack("<II", 0x46554747, 3) + struct.pack("<QQ", 1, 1)
    pre += tiny._str("a", 3) + struct.pack("<II", tiny.U32, 1)
    pre += tiny._str("big", 3) + struct.pack("<I", 2) + struct.pack("<QQ", k, n) + struct.pack("<IQ", 8, 0)
    pre += b"\x00" * ((-len(pre)) % 32)
    p = tmp_path / "big.gguf"
    p.write_bytes(pre + data.tobytes())
    c = Content.read(str(p))
    q = c.tensor("big")
    assert np.array_equal(q.data_.cpu().numpy(), data)
    assert int(q.storage_[nbytes:].abs().sum().item()) == 0


def test_expert_stack_from_the_file_and_stack_some():
    c = Content.read(V3)
    stack = c.tensor("blk.0.ffn_gate_exps.weight")  # [4, 32, 64] MXFP4
    e, n, k = stack.shape
    per = stack.data_.numel() // e
    experts = [QTensor(stack.data_[i * per:(i + 1) * per].clone(), (n, k), stack.dtype) for i in range(e)]
    # stack_some: experts 1 and 3 at slots 0 and 4 of 5; the other slots zero
    some = QTensor.stack_some(5, [(0, experts[1]), (4, experts[3])])
    assert some.shape == (5, n, k)
    assert torch.equal(some.data_[:per], experts[1].data_) and torch.equal(some.data_[4 * per:5 * per], experts[3].data_)
    assert int(some.data_[per:4 * per].abs().sum().item()) == 0
    assert some.padded_bytes() == lib().qmm_padded_bytes(int(stack.dtype), 5 * n * k)
    # a routed product through the loaded stack equals each expert's own forward
    rng = np.random.default_rng(8)
    x = torch.from_numpy(rng.standard_normal((2, k)).astype(np.float32)).cuda()
    ids = torch.tensor([1, 3], dtype=torch.int32, device="cuda")
    sorted_ids = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    y = moe_forward(x, stack, sorted_ids, ids, None, 1)
    for p, ex in ((0, 1), (1, 3)):
        assert torch.equal(y[p], QMatMul(experts[ex]).forward(x[p:p + 1].contiguous())[0])
    with pytest.raises(ValueError):
        QTensor.stack_some(2, [(0, experts[0]), (1, QTensor.quantize(torch.zeros((8, 64), device="cuda"),
                                                                     GgmlDType.Q8_0))])
