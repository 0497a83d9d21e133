"""The Q8_0 hidden-state wire codec on the device against the CPU oracle
(oracle/qref_wire.c, pinned in test_wire_oracle.py): encoded bytes and
decoded values bit for bit, at the sizes a layer split sends (a token's
hidden state of 4096 / 8192 values, a prompt chunk of 512 tokens) and at
lengths that leave a partial trailing group."""
import numpy as np
import pytest
import torch

from helpers import special_rows
from oracle import qref
from swarmllm_amd import quant
from swarmllm_amd._lib import QMM_UNSUPPORTED, lib

pytestmark = pytest.mark.gpu


def inputs(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32)
    ch = rng.permutation(n)[: max(1, n // 100)]
    x[ch] *= np.float32(20.0)
    return x


@pytest.mark.parametrize("n", [1, 31, 32, 33, 50, 4096, 8192, 512 * 4096, 4096 * 3 + 17])
def test_wire_encode_decode_bit_exact(n):
    x = inputs(n, n)
    xt = torch.from_numpy(x).cuda()
    b = quant.quantize_q8_0(xt)
    want = qref.wire_encode(x)
    assert b.numel() == want.size == quant.q8_0_byte_len_checked(n)
    assert np.array_equal(b.cpu().numpy(), want)
    y = quant.dequantize_q8_0(b, n).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), qref.wire_decode(want, n).view(np.uint32))


def test_wire_special_values_bit_exact():
    """Zeros, ties of the rounding, subnormal-scale values, powers of two and
    non-finite values (skipped by the block maximum, coded by the clamp)."""
    sp = special_rows(96).ravel()
    extra = np.array([np.inf, -np.inf, np.nan, 2.5, -2.5, 127.0, 0.5, -0.5] + [1.0] * 24, np.float32)
    allbad = np.array([np.nan, np.inf, -np.inf] * 10 + [np.nan, np.nan], np.float32)
    x = np.concatenate([sp, extra, allbad, np.zeros(7, np.float32)]).astype(np.float32)
    b = quant.quantize_q8_0(torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(b, qref.wire_encode(x))
    y = quant.dequantize_q8_0(torch.from_numpy(b).cuda(), x.size).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), qref.wire_decode(b, x.size).view(np.uint32))


def test_wire_rejects_a_wrong_length_and_takes_empty_input():
    with pytest.raises(ValueError):
        quant.dequantize_q8_0(torch.zeros(33, dtype=torch.uint8, device="cuda"), 32)
    st = lib().qmm_wire_decode(torch.zeros(68, dtype=torch.uint8, device="cuda").data_ptr(), 67, 50,
                               torch.empty(50, device="cuda").data_ptr(), 0)
    assert st == QMM_UNSUPPORTED
    assert quant.quantize_q8_0(torch.empty(0, device="cuda")).numel() == 0
    assert quant.dequantize_q8_0(torch.empty(0, dtype=torch.uint8, device="cuda"), 0).numel() == 0
