"""The Q8_0 hidden-state wire codec on the device, with the names of the
reference's module (src/inference/quant.rs): the bytes in which a layer
split sends activations between the peers that hold consecutive layers.

Per 32 values [f16 scale][32 x i8] = 34 bytes, a partial trailing group
zero-padded; bit-exact to the reference's CPU codec. Runs through libqmm's
qmm_wire_* entry points (no fallback).
"""
from __future__ import annotations

from typing import Optional

import torch

from ._lib import check, lib

GROUP_SIZE = 32
BLOCK_BYTES = 2 + GROUP_SIZE


def q8_0_byte_len_checked(n: int) -> Optional[int]:
    """ceil(n / 32) * 34, or None when it would overflow (q8_0_byte_len_checked,
    src/inference/quant.rs:98-104)."""
    if n < 0:
        return None
    if n == 0:
        return 0
    b = lib().qmm_wire_bytes(n)
    return None if b == 0 else int(b)


def quantize_q8_0(values: torch.Tensor) -> torch.Tensor:
    """The wire bytes (uint8, on values' device) of an f32 tensor, flattened
    (quantize_q8_0, src/inference/quant.rs:24-60)."""
    if values.dtype != torch.float32 or not values.is_cuda:
        raise TypeError("quantize_q8_0 takes an f32 tensor on the GPU")
    x = values.contiguous().view(-1)
    n = x.numel()
    out = torch.empty(q8_0_byte_len_checked(n), dtype=torch.uint8, device=x.device)
    check("qmm_wire_encode", lib().qmm_wire_encode(x.data_ptr() if n else None, n, out.data_ptr() if n else None,
                                                   torch.cuda.current_stream(x.device).cuda_stream))
    return out


def dequantize_q8_0(b: torch.Tensor, num_elements: int) -> torch.Tensor:
    """The f32 values of wire bytes (dequantize_q8_0, src/inference/quant.rs:65-92).
    Raises ValueError when the byte length is not the one num_elements take,
    as the reference returns Err."""
    if b.dtype != torch.uint8 or not b.is_cuda:
        raise TypeError("dequantize_q8_0 takes uint8 bytes on the GPU")
    expected = q8_0_byte_len_checked(num_elements)
    if expected is None or b.numel() != expected:
        raise ValueError(f"Q8_0 byte length mismatch: got {b.numel()}, expected {expected} "
                         f"({num_elements} elements)")
    b = b.contiguous()
    out = torch.empty(num_elements, dtype=torch.float32, device=b.device)
    if num_elements:
        check("qmm_wire_decode", lib().qmm_wire_decode(b.data_ptr(), b.numel(), num_elements, out.data_ptr(),
                                                       torch.cuda.current_stream(b.device).cuda_stream))
    return out
