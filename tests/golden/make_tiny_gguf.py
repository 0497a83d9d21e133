"""Writes the tiny GGUF files the loader tests read (tests/golden/tiny_v3.gguf,
tests/golden/tiny_v1.gguf) and returns what they hold.

The layout follows the GGUF spec as candle's gguf_file::write emits it
(vendor/candle/candle-core/src/quantized/gguf_file.rs:505-560): little
endian; magic, version, tensor count, metadata count; each key/value pair
(string key, u32 value type, value); each tensor info (name, u32 dimension
count, dimensions innermost first, u32 ggml type, u64 offset from the tensor
data); zero padding up to the alignment; the tensor data, each tensor padded
to the alignment. Version 1 writes counts, string and array lengths and
dimensions as u32. The block bytes come from the CPU oracle's quantizer
(oracle/qref.py, bit-exact to the reference's from_float) on seeded normal
values.

Run as a script to rewrite the files:  python tests/golden/make_tiny_gguf.py
"""
from __future__ import annotations

import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import qref  # noqa: E402

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}

# (name, ggml type, shape outermost first)
TENSORS_V3 = [
    ("blk.0.attn_q.weight", 12, (64, 512)),
    ("blk.0.ffn_down.weight", 14, (48, 512)),
    ("token_embd.weight", 8, (40, 96)),
    ("blk.0.ffn_up.weight", 20, (32, 64)),
    ("blk.0.ffn_gate_exps.weight", 39, (4, 32, 64)),
    ("output_norm.weight", 0, (96,)),
    ("rope_freqs", 1, (16,)),
]
TENSORS_V1 = [
    ("w.q4k", 12, (8, 256)),
    ("w.q8_0", 8, (3, 64)),
]


def metadata_v3():
    """(key, value type, value[, element type]) in file order."""
    return [
        ("general.architecture", STRING, "llama"),
        ("general.name", STRING, "tiny\x00\x00"),  # trailing NULs: the reader drops them
        ("general.alignment", U32, 64),
        ("test.u8", U8, 250),
        ("test.i8", I8, -7),
        ("test.u16", U16, 65000),
        ("test.i16", I16, -30000),
        ("test.u32", U32, 4000000000),
        ("test.i32", I32, -2000000000),
        ("test.f32", F32, 0.5),
        ("test.bool", BOOL, True),
        ("test.u64", U64, 18000000000000000000),
        ("test.i64", I64, -9000000000000000000),
        ("test.f64", F64, -1.25e300),
        ("tokenizer.ggml.tokens", ARRAY, ["<s>", "</s>", "hello", "wörld"], STRING),
        ("llama.rope.dimension_sections", ARRAY, [1, 2, 3], I32),
        ("test.f32s", ARRAY, [1.5, -2.0], F32),
        ("test.empty", ARRAY, [], U32),
        ("test.nested", ARRAY, [[1, 2], [3]], ARRAY),
    ]


def metadata_v1():
    return [("general.architecture", STRING, "tiny-v1"), ("test.u32", U32, 7)]


def tensor_bytes(t: int, shape, seed: int) -> bytes:
    n = int(np.prod(shape))
    rng = np.random.default_rng(seed)
    if t == 0:
        return rng.standard_normal(n).astype("<f4").tobytes()
    if t == 1:
        return rng.standard_normal(n).astype("<f2").tobytes()
    k = shape[-1]
    w = (rng.standard_normal(n) * 0.02).astype(np.float32).reshape(-1, k)
    return qref.from_float(t, w).tobytes()


def _str(s: str, version: int) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<I" if version == 1 else "<Q", len(b)) + b


def _count(n: int, version: int) -> bytes:
    return struct.pack("<I" if version == 1 else "<Q", n)


def _value(vt: int, v, version: int, et: int = None) -> bytes:
    if vt == STRING:
        return _str(v, version)
    if vt == ARRAY:
        out = struct.pack("<I", et) + _count(len(v), version)
        inner = U32 if et == ARRAY else None
        for x in v:
            out += _value(et, x, version, inner)
        return out
    return struct.pack(_FMT[vt], int(v) if vt not in (F32, F64) else v)


def build(version: int, metadata, tensors, alignment: int):
    """The file's bytes, and each tensor's (offset, bytes)."""
    head = struct.pack("<II", 0x46554747, version) + _count(len(tensors), version) + _count(len(metadata), version)
    for item in metadata:
        key, vt, v = item[:3]
        et = item[3] if len(item) > 3 else None
        head += _str(key, version) + struct.pack("<I", vt) + _value(vt, v, version, et)
    datas, offset, infos = [], 0, []
    for i, (name, t, shape) in enumerate(tensors):
        b = tensor_bytes(t, shape, seed=1000 + i)
        head += _str(name, version) + struct.pack("<I", len(shape))
        for d in reversed(shape):
            head += struct.pack("<I" if version == 1 else "<Q", d)
        head += struct.pack("<IQ", t, offset)
        infos.append((offset, b))
        datas.append(b + b"\x00" * ((-len(b)) % alignment))
        offset += len(datas[-1])
    pad = (-len(head)) % alignment
    return head + b"\x00" * pad + b"".join(datas), infos, len(head) + pad


def files():
    """{file name: (bytes, tensor infos, data offset, metadata, tensors)}."""
    v3, i3, o3 = build(3, metadata_v3(), TENSORS_V3, 64)
    v1, i1, o1 = build(1, metadata_v1(), TENSORS_V1, 32)
    return {"tiny_v3.gguf": (v3, i3, o3, metadata_v3(), TENSORS_V3),
            "tiny_v1.gguf": (v1, i1, o1, metadata_v1(), TENSORS_V1)}


if __name__ == "__main__":
    for name, (data, *_rest) in files().items():
        with open(os.path.join(HERE, name), "wb") as f:
            f.write(data)
        print(f"wrote {name}: {len(data)} bytes")
